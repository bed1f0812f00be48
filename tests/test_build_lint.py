"""Static checks of the gfx950 code objects -- CPU only (hipcc cross-compiles).

* No kernel makes a device-function call: the balanced kernel reads its arguments through the
  kernarg-segment pointer, which is only valid in the kernel body (in a called function it is
  null), and calls would also cost registers and latency in the hot loop.
* No packed-FP32 instructions are emitted (the build disables them).
* No kernel spills registers to scratch.
* M0 is written only by the key-split prefix kernel's direct global->LDS loads (cascade.hip
  issues them from inline asm that sets M0 and declares it clobbered): every M0 reference is
  such a write, followed by the wait state and the load, so no compiler-generated code holds a
  value in M0 across them.

Every .hip source of the library is checked.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cuda-kernel-lab_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only"]


def _asm(name, tmp_path):
    out = tmp_path / (name + ".s")
    subprocess.run([HIPCC, *FLAGS, "-S", os.path.join(CSRC, name + ".hip"), "-o", str(out)],
                   check=True, stderr=subprocess.DEVNULL)
    return out.read_text()


SOURCES = sorted(f[:-4] for f in os.listdir(CSRC) if f.endswith(".hip"))


def test_every_source_is_linted():
    assert {"decode", "cascade", "append", "misc", "noalloc"} <= set(SOURCES)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("name", SOURCES)
def test_no_calls_no_packed_fp32(name, tmp_path):
    asm = _asm(name, tmp_path)
    assert "s_swappc_b64" not in asm, f"{name}.hip: a kernel calls a device function"
    assert not re.search(r"\bv_pk_(add|mul|fma)_f32\b", asm), f"{name}.hip: packed FP32 emitted"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("name", SOURCES)
def test_no_scratch_spills(name, tmp_path):
    out = subprocess.run([HIPCC, *FLAGS, "-c", os.path.join(CSRC, name + ".hip"), "-o", str(tmp_path / "d.o"),
                          "-Rpass-analysis=kernel-resource-usage"], capture_output=True, text=True)
    text = out.stderr
    names = re.findall(r"Function Name: (\S+)", text)
    spills = re.findall(r"VGPRs Spill: (\d+)", text)
    sspills = re.findall(r"SGPRs Spill: (\d+)", text)
    assert len(names) == len(spills) == len(sspills)
    if name != "noalloc":   # (noalloc.hip holds a device array and host code, no kernel)
        assert names
    for n, sp, ss in zip(names, spills, sspills):
        assert int(sp) == 0 and int(ss) == 0, f"{name}.hip: {n} spills {sp} VGPRs, {ss} SGPRs"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_m0_only_for_direct_lds_loads(tmp_path):
    asm = _asm("cascade", tmp_path)
    lines = [ln.split(";")[0].strip() for ln in asm.splitlines()]
    lines = [ln for ln in lines if ln]
    uses = [i for i, ln in enumerate(lines) if re.search(r"\bm0\b", ln)]
    loads = sum(1 for ln in lines if ln.startswith("global_load_lds_dwordx4"))
    assert uses and len(uses) == loads
    for i in uses:
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", lines[i]), lines[i]
        assert lines[i + 1] == "s_nop 0" and lines[i + 2].startswith("global_load_lds_dwordx4"), lines[i:i + 3]
