"""Build-time guards of the persistent decode kernel's tuning knobs (no GPU).

The loader streams a compute wave's units into a ring of LDS slots, and the compute wave waits for every line of
a unit before it releases any of them. A configuration whose units do not fit the ring would leave the wave
waiting for lines the loader can never publish. decode.hip rejects such a configuration with a static_assert.
These tests front-end-compile the kernel (hipcc -fsyntax-only, about a second each) for the default, for every
configuration the sweep builds, and for configurations that must be refused.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

from cudallm_amd.sweep_decode import configs

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else None)
pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")


def front_end(defines: dict) -> subprocess.CompletedProcess:
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "--offload-device-only", "-fsyntax-only",
           f"-I{ROOT / 'include'}", f"-I{ROOT / 'cudallm_amd' / 'csrc'}",
           *(f"-D{k}={v}" for k, v in defines.items()), str(ROOT / "cudallm_amd" / "csrc" / "kernels" / "decode.hip")]
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("name", sorted(configs()))
def test_sweep_configurations_pass_the_guards(name):
    r = front_end(configs()[name])
    assert r.returncode == 0, f"{name}: {r.stderr[-2000:]}"


@pytest.mark.parametrize("defines, message", [
    # 16 int8 lm_head rows of 2 lines each are 32 lines, more than 22 slots
    ({"CLLM_LM_ROWS_QUANT": 16}, "a unit's lines fit the ring"),
    # a bf16 lm_head unit of 8 rows is 32 lines, more than 30 slots
    ({"CLLM_LM_ROWS_BF16": 8}, "a unit's lines fit the ring"),
    # two int8 down rows (8 lines each) are read as one unit
    ({"CLLM_RING_SLOTS_QUANT": 14}, "two int8 down rows fit the ring"),
])
def test_units_that_do_not_fit_the_ring_are_refused(defines, message):
    r = front_end(defines)
    assert r.returncode != 0
    assert message in r.stderr, r.stderr[-2000:]


def makefile_decode_command(obj: Path) -> list[str]:
    """The Makefile's own compile command for the decode kernel (make -n), writing `obj`."""
    r = subprocess.run(["make", "-n", "-B", "-C", str(ROOT / "cudallm_amd"), f"BUILD={obj.parent}", str(obj)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    line = next(ln for ln in r.stdout.splitlines() if "decode.hip" in ln and "hipcc" in ln)
    return line.split()


def test_decode_kernels_use_no_scratch(tmp_path):
    """The decode kernel, built exactly as the Makefile builds it, must keep every value in registers: no VGPR
    spills and no scratch memory for any weight type.  The one build that miscomputed int4 results (layer 1's SwiGLU
    outputs wrong in every workgroup, varying from run to run, cause not found) was the only one that spilled, and
    the kernel sits at 252-254 of its 256 VGPRs, so a change that tips it into spills must fail here first."""
    cmd = makefile_decode_command(tmp_path / "decode.o") + ["-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600, cwd=ROOT / "cudallm_amd")
    assert r.returncode == 0, r.stderr[-2000:]
    kernels = {}
    name = None
    for ln in r.stderr.splitlines():
        if "Function Name:" in ln:
            name = ln.split("Function Name:")[1].split()[0]
        elif name and "remark:" in ln:
            key, _, val = ln.split("remark:")[1].strip().partition(":")
            kernels.setdefault(name, {})[key.strip()] = val.split("[")[0].strip()
    decode = {k: v for k, v in kernels.items() if "decode_kernel" in k}
    assert len(decode) == 3, sorted(kernels)
    for k, v in decode.items():
        assert v["ScratchSize [bytes/lane]"] == "0", (k, v)
        assert v["VGPRs Spill"] == "0", (k, v)
        assert int(v["VGPRs"]) <= 256, (k, v)
