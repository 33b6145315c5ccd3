"""ISA checks of the decode-step in-projection (gdn_decode_skinny_kernel<0, *>)
in gdn_18646_amd/csrc/layer.hip, on the CPU (hipcc cross-compiles gfx950).

The kernel copies x and gamma to LDS with global_load_lds, then issues the
epilogue's EPI small loads (conv taps, cache window, x_n history) and its
MAXSTEPS weight loads, then waits with vmcnt(MAXSTEPS + EPI): vector memory
operations retire in issue order, so that wait covers the LDS copies only if
exactly MAXSTEPS + EPI vector memory operations sit between the last copy and
the wait.  A compiler that moved another load (or a spill) into that window
would let RMSNorm read LDS before the copy lands; this test fails first.
"""

import os
import re
import shutil
import subprocess

import pytest

HIPCC = "/opt/rocm/bin/hipcc"
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "gdn_18646_amd", "csrc", "layer.hip")

VMEM = re.compile(r"^\s*(buffer|global|scratch|flat)_(load|store|atomic)")


@pytest.fixture(scope="module")
def layer_asm(tmp_path_factory):
    if not shutil.which(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "layer.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", SRC, "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def _function(asm, symbol):
    start = asm.index(f"\n{symbol}:")
    return asm[start:asm.index("s_endpgm", start)].splitlines()


@pytest.mark.parametrize("maxsteps", [8, 16])
def test_in_proj_dma_wait_covers_only_the_weight_loads(layer_asm, maxsteps):
    sym = f"_ZN12_GLOBAL__N_124gdn_decode_skinny_kernelILi0ELi{maxsteps}EEEvNS_12SkinnyParamsE"
    body = _function(layer_asm, sym)
    last_dma = max(i for i, ln in enumerate(body) if "global_load_lds_dwordx4" in ln)
    wait = next(i for i in range(last_dma, len(body)) if re.search(r"s_waitcnt vmcnt\(\d+\)", body[i]))
    n = int(re.search(r"vmcnt\((\d+)\)", body[wait]).group(1))
    between = [ln.strip() for ln in body[last_dma + 1:wait] if VMEM.match(ln)]
    epi = 9  # kEpiLoads in layer.hip: 7 global_load_ushort + 2 global_load_dwordx4
    assert n == maxsteps + epi, f"first wait after the copies is vmcnt({n}), expected vmcnt({maxsteps + epi})"
    assert len(between) == maxsteps + epi, between
    assert sum(ln.startswith("buffer_load_dwordx4") for ln in between) == maxsteps, between
    assert all(ln.startswith(("buffer_load_dwordx4", "global_load_ushort", "global_load_dwordx4")) for ln in between)
    assert not any("scratch_" in ln for ln in body), "the kernel spills"


def test_tile_kernels_keep_their_ring_waits_and_do_not_spill(layer_asm):
    """The decode-step tile kernels (gdn_decode_tile_kernel<MODE, NC, TN>)
    order their LDS ring by explicit vmcnt waits that count the copies a
    slice issues (two per wave: one of A, one of W, also for 32-wide tiles,
    whose W copy runs on lanes 0..31 of every wave): vmcnt(6) after the four
    slots are issued and vmcnt(4) in the loop.  Every instantiation must keep
    both waits, issue its copies as global_load_lds_dwordx4 only, and not
    spill (a spill's scratch access inside the loop would shift the count)."""
    syms = sorted(set(re.findall(r"^(_ZN12_GLOBAL__N_122gdn_decode_tile_kernel\w+):", layer_asm, re.M)))
    assert len(syms) == 9, syms  # in-projection NC 0..3 x TN 32, 64; out-projection TN 32
    for sym in syms:
        body = _function(layer_asm, sym)
        text = "\n".join(body)
        assert "scratch_" not in text, f"{sym} spills"
        waits = re.findall(r"s_waitcnt vmcnt\((\d+)\)", text)
        assert "6" in waits and "4" in waits, (sym, waits)
        assert any("global_load_lds_dwordx4" in ln for ln in body), sym
        assert not any(re.search(r"global_load_lds_dword(x2|x3)?\s", ln) for ln in body), sym
