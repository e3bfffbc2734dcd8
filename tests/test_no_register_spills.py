"""Every gfx950 kernel of the device library keeps its state in registers:
each translation unit is compiled to device assembly with the build's own
flags, and every kernel descriptor must show no private (scratch) segment,
that is no register spills. CPU only (hipcc cross-compiles)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from mitten_amd import _build

KERNEL = re.compile(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", re.S)
SCRATCH = re.compile(r"\.amdhsa_private_segment_fixed_size (\d+)")


def _device_asm(src: str, out: str) -> subprocess.CompletedProcess:
    cmd = _build.device_obj_cmd(src, out)
    i = cmd.index("-c")
    cmd[i:i + 1] = ["--cuda-device-only", "-S"]
    return subprocess.run(cmd, capture_output=True, text=True)


def test_no_kernel_spills_registers(tmp_path):
    hipcc = _build._hipcc()
    if not (os.path.exists(hipcc) or shutil.which(hipcc)):
        pytest.skip("hipcc is not available")
    outs = {s: str(tmp_path / (os.path.splitext(s)[0] + ".s")) for s in _build.DEVICE_SOURCES}
    with ThreadPoolExecutor(len(outs)) as ex:
        results = dict(zip(outs, ex.map(lambda s: _device_asm(s, outs[s]), outs)))
    spills, kernels = [], 0
    for src, res in results.items():
        assert res.returncode == 0, f"{src}: {res.stderr[-2000:]}"
        for name, body in KERNEL.findall(open(outs[src]).read()):
            kernels += 1
            m = SCRATCH.search(body)
            if m and int(m.group(1)) > 0:
                spills.append(f"{src}: {name} ({m.group(1)} bytes per lane)")
    assert kernels > 0
    assert not spills, "kernels with register spills:\n" + "\n".join(spills)
