"""The ctypes mirror of `DuckServoSubstep` (duck_gym_amd/native.py) has the
size and field offsets the C compiler gives include/duck_hip.h's struct."""

import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from duck_gym_amd.native import DuckServoSubstep

ROOT = Path(__file__).resolve().parents[1]
FIELDS = [name for name, _ in DuckServoSubstep._fields_]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc absent")
def test_servo_substep_struct_layout(tmp_path):
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof(DuckServoSubstep, {f}));' for f in FIELDS)
    src = tmp_path / "layout.c"
    src.write_text(f"""#include <stddef.h>
#include <stdio.h>
#include "duck_hip.h"
int main(void) {{
  printf("size %zu\\n", sizeof(DuckServoSubstep));
{body}
  return 0;
}}
""")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    assert int(out["size"]) == ctypes.sizeof(DuckServoSubstep)
    for f in FIELDS:
        assert int(out[f]) == getattr(DuckServoSubstep, f).offset, f
