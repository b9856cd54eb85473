"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, as the
reference's DUCK_SANITIZE build runs its CPU code (CMakeLists.txt:6-14):
tests/native/sanitize_driver.cpp links the product's `.duck` loader
(duck_gym_amd/csrc/duck_model.cpp) and the CPU oracle with
-fsanitize=address,undefined, then loads every malformed and valid model of
the test corpus and steps the valid ones in both oracle modes and both
precisions.  Any sanitizer report fails the run (halt_on_error)."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from model_text import caterpillar
from test_model_errors import RUNTIME, VALUE

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="g++ absent")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    out = tmp_path_factory.mktemp("sanitize") / "sanitize_driver"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           str(ROOT / "tests" / "native" / "sanitize_driver.cpp"),
           str(ROOT / "duck_gym_amd" / "csrc" / "duck_model.cpp"),
           str(ROOT / "oracle" / "avbd_oracle.cpp"), "-o", str(out), "-pthread"]
    subprocess.run(cmd, check=True)
    return out


def _run(driver, *args):
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    out = subprocess.run([str(driver), *map(str, args)], capture_output=True, text=True,
                         env=env, timeout=600)
    assert out.returncode == 0 and "Sanitizer" not in out.stderr, out.stdout[-2000:] + out.stderr
    return out.stdout


def _valid_models(models, tmp_path):
    from duck_gym_amd import duck_format as D
    from test_gpu_shapes import CASES, mixed_mjcf

    paths = [models[k] for k in ("standing", "selfc", "friction", "limp")]
    paths.append(GOLDEN / "pendulum.duck")
    (tmp_path / "caterpillar.duck").write_text(caterpillar())
    paths.append(tmp_path / "caterpillar.duck")
    for name, (tail, pairs, _) in CASES.items():
        model = D.from_mjcf(mixed_mjcf(tail))
        if pairs:
            model = D.with_body_pairs(model)
        D.write_duck(model, tmp_path / f"mixed_{name}.duck")
        paths.append(tmp_path / f"mixed_{name}.duck")
    return paths


def test_loader_under_sanitizers(driver, models, tmp_path):
    bad = []
    for i, (name, text, message) in enumerate(RUNTIME + [c for c in VALUE if c[1]]):
        path = tmp_path / f"bad{i}.duck"
        path.write_text(text)
        bad.append((path, message))
    out = _run(driver, "load", *[p for p, _ in bad], tmp_path / "absent.duck",
               *_valid_models(models, tmp_path))
    lines = out.splitlines()
    for (path, message), line in zip(bad, lines):
        assert line.startswith("error") and message in line, (path, line)
    assert lines[len(bad)].startswith("error") and "Cannot read model" in lines[len(bad)]
    assert all(line.startswith("ok") for line in lines[len(bad) + 1:])


def test_oracle_under_sanitizers(driver, models, tmp_path):
    paths = _valid_models(models, tmp_path)
    out = _run(driver, "step", *paths)
    lines = out.splitlines()
    rejected = sum(line.startswith("rejected") for line in lines)
    stepped = sum(line.startswith("stepped") for line in lines)
    assert all("mode 1" in line and "Body contacts" in line
               for line in lines if line.startswith("rejected"))
    assert stepped + rejected == 4 * len(paths) and "convex query ok" in out
    assert stepped >= 2 * len(paths)
    # the threaded batch driver, both precisions of every model
    assert sum(line.startswith("batch stepped") for line in lines) == 2 * len(paths)
