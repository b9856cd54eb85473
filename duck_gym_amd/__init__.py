"""MI355X-native (gfx950 HIP) batched rigid-body AVBD environment step.

Drop-in for duck_gym's native batch (`CudaBatch`, src/cuda/extension.cu) and
its tensor VecEnv (`TensorEnv`, python/duck_gym/tensor_env.py).
"""

from .native import CudaBatch, library  # noqa: F401


def build():
    """Compile the HIP library and return a module-like object exposing
    `CudaBatch`, the role scripts/build_cuda.py:build() plays for
    python/duck_gym/tensor_env.py:95-101."""
    from . import hipbuild as _build
    import sys

    _build.build(force=False)
    return sys.modules[__name__]
