"""Host-side checks that need no GPU: the C-ABI library loads and exports
every entry point include/duck_hip.h declares, the synthetic MicroDuck-like
model satisfies the reference's model contract, and the state codec
round-trips."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from duck_gym_amd import native
from duck_gym_amd.microduck import HOME, JOINT_NAMES, model_text
from oracle.oracle import Oracle, ReferenceProbe, probe_available

ROOT = Path(__file__).resolve().parents[1]


def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "duck_hip.h").read_text()
    declared = set(re.findall(r"\b(duck_[a-z_]+)\s*\(", header))
    assert len(declared) >= 17
    lib = ctypes.CDLL(str(native.LIBRARY))  # loading needs no GPU
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(native.EXPORTED)


def test_microduck_model_contract():
    """16 bodies, 14 hinges in the order of src/cuda/extension.cu:228-231,
    parent before child with a < b, masses 0.02-0.4 kg, a bipartite tree and
    contact capacity <= 64 (src/cuda/model.hpp:26-91)."""
    text, meta = model_text()
    lines = text.splitlines()
    head = lines[0].split()
    assert head[:2] == ["DUCK_MODEL", "1"] and head[2:] == ["16", "14", "15"]
    bodies = [l.split() for l in lines[2:18]]
    joints = [l.split() for l in lines[18:32]]
    shapes = [l.split() for l in lines[32:47]]
    assert [j[0] for j in joints] == list(JOINT_NAMES) == meta["joint_names"]
    masses = [float(b[1]) for b in bodies[1:]]
    assert min(masses) >= 0.02 and max(masses) <= 0.4
    seen = {1}
    colour = {0: 0, 1: 0}
    for j in joints:
        a, b = int(j[1]), int(j[2])
        assert a < b and a in seen and b not in seen
        seen.add(b)
        colour[b] = 1 - colour[a]
    assert seen == set(range(1, 16))
    assert sum(1 for c in colour.values() if c == 0) - 2 == 6  # 7 dynamic + world + root
    assert 4 * len(shapes) <= 64
    feet = [s for s in shapes if s[1] == "3"]
    assert len(feet) == 2 and all(int(s[13]) == 8 for s in feet)  # 8-vertex hulls
    sc_text, sc_meta = model_text(self_contact=True)
    assert 4 * 15 + int(sc_text.splitlines()[47]) <= 64 and sc_meta["self_contact"]


@pytest.mark.skipif(not probe_available(), reason="reference build (oracle/_ref) absent")
def test_microduck_model_loads_in_reference_and_stands(models):
    home = np.array([HOME[n] for n in JOINT_NAMES])
    for fp64 in (False, True):
        p = ReferenceProbe(models["standing"], 0.005, 10, fp64)
        p.reset(home)
        for _ in range(200):
            p.step(home, None, 1, 8.0, 0.0)
        b, j, d = p.snapshot()
        assert not d[5] and d[2] == 8  # both feet flat: 4 + 4 ground contacts
        assert 0.20 < b[1, 2] < 0.23  # root COM stays near its HOME height


def test_oracle_rejects_invalid_models(tmp_path):
    bad = {
        "header": "DUCK_MODEL 3 2 0 0\n0 0 -9.81 0\n",
        "truncated": "DUCK_MODEL 1 2 0 0\n0 0 -9.81 0\nworld 0 0 0 0 0 0 0 1 0 0 0\n",
        "mass": "DUCK_MODEL 1 2 0 0\n0 0 -9.81 0\nworld 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0\n"
                "b 1 0 1 1 0 0 0 1 0 0 0 0 0 0 0 0 0\n",
    }
    for name, text in bad.items():
        path = tmp_path / f"{name}.duck"
        path.write_text(text)
        with pytest.raises(ValueError):
            Oracle(path)


def test_state_codec_round_trip():
    from duck_gym_amd.state import FIELDS, StateCodec

    # A synthetic layout: B=4, J=2, CG=3, CS=2, float64.
    layout = dict(B=4, J=2, CG=3, CS=2, real=8, blob=4096, header=0)
    off = 0

    def take(n):
        nonlocal off
        o = off
        off += n
        return o

    for name, k in (("x", 3 * 4), ("q", 4 * 4), ("v", 3 * 4), ("w", 3 * 4), ("mass", 4),
                    ("inertia", 12), ("force", 3), ("lambda", 14), ("penalty", 14),
                    ("lambdaF", 2), ("penaltyF", 2), ("target", 2), ("kp", 2),
                    ("maxTorque", 2), ("torque", 2), ("frictionloss", 2), ("damping", 2),
                    ("diag", 8), ("friction", 1)):
        layout[name] = take(8 * k)
    for name in ("failed", "ngc", "nsc", "colorCount"):
        layout[name] = take(4)
    layout["colors"] = take(16)
    layout["header"] = off
    layout["gc"], layout["gcBytes"] = take(3 * 104), 104
    layout["sc"], layout["scBytes"] = take(2 * 192), 192
    for i, name in enumerate(("gc_id", "gc_local", "gc_anchor", "gc_c0", "gc_lambda", "gc_penalty")):
        layout[name] = [0, 8, 32, 48, 56, 80][i]
    for i, name in enumerate(("sc_id", "sc_local", "sc_localB", "sc_t1", "sc_t2", "sc_n", "sc_c0",
                              "sc_friction", "sc_lambda", "sc_penalty")):
        layout[name] = [0, 8, 32, 56, 80, 104, 128, 136, 144, 168][i]
    codec = StateCodec([layout[f] for f in FIELDS], bodies=3, joints=2)
    rng = np.random.default_rng(0)
    s = {k: rng.normal(size=shape) for k, shape in (
        ("x", (3, 3)), ("q", (3, 4)), ("v", (3, 3)), ("w", (3, 3)), ("mass", (3,)),
        ("inertia", (3, 3)), ("lambda", (2, 7)), ("penalty", (2, 7)), ("lambdaF", (2,)),
        ("penaltyF", (2,)), ("target", (2,)), ("kp", (2,)), ("maxTorque", (2,)),
        ("torque", (2,)), ("frictionloss", (2,)), ("damping", (2,)), ("force", (3,)),
        ("diag", (8,)))}
    s.update(friction=0.7, failed=1, ngc=1, nsc=1, colorCount=3, colors=np.array([0, 1, 2]))
    s["gc"] = [dict(id=5 | (2 << 6) | (7 << 12), local=rng.normal(size=3), anchor=rng.normal(size=2),
                    c0=rng.normal(size=1), penalty=rng.normal(size=3), **{"lambda": rng.normal(size=3)})]
    s["sc"] = [dict(id=1 | (2 << 6) | (3 << 12) | (4 << 18), **{k: rng.normal(size=n) for k, n in (
        ("local", 3), ("localB", 3), ("t1", 3), ("t2", 3), ("n", 3), ("c0", 1), ("friction", 1),
        ("lambda", 3), ("penalty", 3))})]
    raw = np.zeros(layout["blob"], np.uint8)
    codec.encode(raw, s)
    out = codec.decode(raw)
    for k in ("x", "q", "lambda", "penalty", "damping", "force", "diag", "colors"):
        np.testing.assert_array_equal(out[k], s[k])
    assert out["failed"] == 1 and out["colorCount"] == 3 and out["friction"] == 0.7
    g = out["gc"][0]
    assert (g["shape"], g["body"], g["feature"], g["stick"]) == (5, 2, 7, False)
    np.testing.assert_array_equal(g["lambda"], s["gc"][0]["lambda"])
    c = out["sc"][0]
    assert (c["body"], c["other"], c["shape"], c["otherShape"]) == (1, 2, 3, 4)
    np.testing.assert_array_equal(c["n"], s["sc"][0]["n"])


def test_ctypes_structs_match_the_c_header(tmp_path):
    """DuckTask / DuckServo field offsets in ctypes equal the C layout."""
    import shutil
    import subprocess

    from duck_gym_amd.native import DuckServo, DuckTask

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "duck_hip.h"', "int main(void){"]
    for struct, cls in (("DuckTask", DuckTask), ("DuckServo", DuckServo)):
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        for name, _ in cls._fields_:
            lines.append(f'printf("{struct}.{name} %zu\\n", offsetof({struct}, {name}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for struct, cls in (("DuckTask", DuckTask), ("DuckServo", DuckServo)):
        assert int(got[struct]) == ctypes.sizeof(cls)
        for name, _ in cls._fields_:
            assert int(got[f"{struct}.{name}"]) == getattr(cls, name).offset, (struct, name)
