"""CPU checks of the drop-in boundary: the C ABI library and the torch binding.

No kernel is launched: the library loads, exports every entry point that
include/gdn_amd.h declares, its pure-host functions answer, and argument
validation rejects bad calls before any HIP call is made.
"""

import os
import re

import pytest
import torch

from gdn_18646_amd import abi, compile_kernels
from gdn_18646_amd.abi import GdnError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "gdn_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = abi.load()
    names = _declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/gdn_amd.h but not exported"
    assert set(names) == set(abi.SIGNATURES), "abi.SIGNATURES out of sync with the header"


def test_host_functions():
    lib = abi.load()
    assert lib.gdn_abi_version() == 1
    assert lib.gdn_status_string(0) == b"ok"
    assert lib.gdn_status_string(3) == b"workspace too small"
    # dv a multiple of 128: 8 KiB per (chunk, head), the six nonzero Tp fragments, the
    # gate block and the token block (1 KiB each); the metric shape has 128 chunks x 16
    # heads.  With only 16 (sequence, head) pairs the state pass splits each sequence into
    # 16 chunk groups, each with a 128 x dv fp32 zero-state result and a 128 x 128 bf16
    # transition.
    b = lib.gdn_prefill_workspace_bytes(1, 16, 8192, 128, 128)
    per_chunk = 2048 * (6 + 1 + 1) * 1024
    groups = 16 * 16 * (128 * 128 * 4 + 128 * 128 * 2)
    assert per_chunk + groups <= b < per_chunk + groups + 8192
    # enough (sequence, head) pairs to fill the chip: no groups
    b = lib.gdn_prefill_workspace_bytes(16, 16, 8192, 128, 128)
    assert 16 * per_chunk <= b < 16 * per_chunk + 8192
    assert lib.gdn_prefill_workspace_bytes(1, 16, 0, 128, 128) == 0
    # other dv: 13 KiB records, the six Aq fragments in place of the token block
    assert lib.gdn_prefill_varlen_workspace_bytes(3, 2, 130, 128, 64) >= (130 // 64 + 3) * 2 * 13 * 1024
    assert lib.gdn_prefill_workspace_bytes(1, 2, 640, 128, 64) >= 10 * 2 * 13 * 1024


FAKE = 4096  # non-null, 16-byte aligned; validation fails before it is ever dereferenced


def test_prefill_noalloc_refuses_oversized_shape():
    """The static scratch limit is checked before any HIP call (none runs here)."""
    with pytest.raises(GdnError, match="WORKSPACE.*static buffer"):
        abi.call("gdn_prefill_noalloc_hip", *([FAKE] * 5), 0.0, FAKE, FAKE, None, 0.0, FAKE, FAKE,
                 4, 16, 8192, 128, 128, None)
    with pytest.raises(GdnError, match="UNSUPPORTED.*dk=64"):
        abi.call("gdn_prefill_noalloc_hip", *([FAKE] * 5), 0.0, FAKE, FAKE, None, 0.0, FAKE, FAKE,
                 1, 16, 64, 64, 128, None)


def test_decode_validation_errors():
    with pytest.raises(GdnError, match="UNSUPPORTED.*dk=64"):
        abi.call("gdn_decode_hip", *([FAKE] * 8), 0.1, FAKE, FAKE, 2, 2, 64, 128, None)
    with pytest.raises(GdnError, match="UNSUPPORTED.*dv=48"):
        abi.call("gdn_decode_hip", *([FAKE] * 8), 0.1, FAKE, FAKE, 2, 2, 128, 48, None)
    with pytest.raises(GdnError, match="INVALID_ARGUMENT.*null"):
        abi.call("gdn_decode_hip", None, *([FAKE] * 7), 0.1, FAKE, FAKE, 2, 2, 128, 128, None)
    with pytest.raises(GdnError, match="alignment"):
        abi.call("gdn_decode_hip", FAKE + 2, *([FAKE] * 7), 0.1, FAKE, FAKE, 2, 2, 128, 128, None)
    # B == 0 is a valid no-op
    abi.call("gdn_decode_hip", *([None] * 8), 0.1, None, None, 0, 2, 128, 128, None)


def test_prefill_validation_errors():
    args = [FAKE] * 5 + [0.0, FAKE, None, None, 0.0, FAKE, FAKE]
    with pytest.raises(GdnError, match="UNSUPPORTED.*dv=40"):
        abi.call("gdn_prefill_hip", *args, 1, 2, 64, 128, 40, FAKE, 1 << 20, None)
    with pytest.raises(GdnError, match="UNSUPPORTED.*dk=256"):
        abi.call("gdn_prefill_hip", *args, 1, 2, 64, 256, 128, FAKE, 1 << 20, None)
    with pytest.raises(GdnError, match="WORKSPACE"):
        abi.call("gdn_prefill_hip", *args, 1, 2, 64, 128, 128, FAKE, 16, None)
    with pytest.raises(GdnError, match="WORKSPACE"):
        abi.call("gdn_prefill_hip", *args, 1, 2, 64, 128, 128, None, 1 << 30, None)
    with pytest.raises(GdnError, match="INVALID_ARGUMENT"):
        abi.call("gdn_prefill_varlen_hip", *([FAKE] * 5), 0.0, FAKE, None, None, 3, 0, None, 0.0, FAKE, FAKE,
                 2, 64, 128, 128, FAKE, 1 << 30, None)


def test_support_validation_errors():
    with pytest.raises(GdnError, match="multiple of 8"):
        abi.call("gdn_rmsnorm_hip", FAKE, FAKE, FAKE, 4, 100, 1e-6, None)
    with pytest.raises(GdnError, match="multiple of 64"):
        abi.call("gdn_proj_conv_silu_hip", FAKE, FAKE, FAKE, FAKE, 1, 8, 100, 64, 4, None)
    with pytest.raises(GdnError, match="conv_k"):
        abi.call("gdn_proj_conv_silu_hip", FAKE, FAKE, FAKE, FAKE, 1, 8, 128, 64, 5, None)


def test_decode_projection_validation_errors():
    in_args = lambda B, D, ck: ([FAKE, FAKE, 1e-6] + [FAKE] * 11 + [B, D, 2, 128, 128, ck, None])
    with pytest.raises(GdnError, match="UNSUPPORTED.*B=17"):
        abi.call("gdn_decode_in_proj_hip", *in_args(17, 2048, 4))
    with pytest.raises(GdnError, match="UNSUPPORTED.*D=100"):
        abi.call("gdn_decode_in_proj_hip", *in_args(4, 100, 4))
    with pytest.raises(GdnError, match="UNSUPPORTED.*D=8192"):
        abi.call("gdn_decode_in_proj_hip", *in_args(4, 8192, 4))
    with pytest.raises(GdnError, match="conv_k"):
        abi.call("gdn_decode_in_proj_hip", *in_args(4, 2048, 5))
    with pytest.raises(GdnError, match="INVALID_ARGUMENT.*null"):
        abi.call("gdn_decode_in_proj_hip", None, *in_args(4, 2048, 4)[1:])
    abi.call("gdn_decode_in_proj_hip", *in_args(0, 2048, 4))  # B == 0: no-op
    with pytest.raises(GdnError, match="UNSUPPORTED.*B=17"):
        abi.call("gdn_decode_out_proj_hip", FAKE, FAKE, FAKE, 17, 2048, 2048, None)
    with pytest.raises(GdnError, match="UNSUPPORTED.*K=2050"):
        abi.call("gdn_decode_out_proj_hip", FAKE, FAKE, FAKE, 4, 2050, 2048, None)
    with pytest.raises(GdnError, match="alignment"):
        abi.call("gdn_decode_out_proj_hip", FAKE + 4, FAKE, FAKE, 4, 2048, 2048, None)


def test_decode_conv_step_validation_errors():
    args = lambda B, D, ck, hist: ([FAKE] * 5 + [FAKE, FAKE if hist else None] + [FAKE] * 5 + [B, D, 2, 128, 64, ck, None])
    with pytest.raises(GdnError, match="B=70000, at most 65535"):
        abi.call("gdn_decode_conv_step_hip", *args(70000, 256, 4, True))
    with pytest.raises(GdnError, match="D=0"):
        abi.call("gdn_decode_conv_step_hip", *args(4, 0, 4, True))
    with pytest.raises(GdnError, match="conv_k=5"):
        abi.call("gdn_decode_conv_step_hip", *args(4, 256, 5, False))
    abi.call("gdn_decode_conv_step_hip", *args(0, 256, 4, True))  # B == 0: no-op


def test_decode_step_validation_errors():
    """The fused step checks every stage's arguments before its first launch."""
    step_args = lambda B, D, dv: ([FAKE, FAKE, 1e-6] + [FAKE] * 10 + [0.1] + [FAKE] * 8 + [B, D, 2, 128, dv, 4, None])
    with pytest.raises(GdnError, match="decode_step: B=65536, at most 65535"):
        abi.call("gdn_layer_decode_step_hip", *step_args(65536, 2048, 128))
    # B > 16: the tiled path's own checks
    with pytest.raises(GdnError, match="decode_step: D=100 must be a multiple of 64"):
        abi.call("gdn_layer_decode_step_hip", *step_args(65, 100, 128))
    with pytest.raises(GdnError, match="decode_step: H dk=256 and H dv=32 must be multiples of 64"):
        abi.call("gdn_layer_decode_step_hip", *step_args(65, 2048, 16))
    tiled_misaligned = step_args(65, 2048, 128)
    tiled_misaligned[21] = FAKE + 4  # y
    with pytest.raises(GdnError, match="decode_step: x/gamma/W/W_o/y"):
        abi.call("gdn_layer_decode_step_hip", *tiled_misaligned)
    tiled_misaligned = step_args(65, 2048, 128)
    tiled_misaligned[11] = FAKE + 4  # S_in: refused by the recurrence's checks, still before any launch
    with pytest.raises(GdnError, match="decode: q/k/S/o need 16-byte"):
        abi.call("gdn_layer_decode_step_hip", *tiled_misaligned)
    with pytest.raises(GdnError, match="decode_in_proj.*D=100"):
        abi.call("gdn_layer_decode_step_hip", *step_args(4, 100, 128))
    abi.call("gdn_layer_decode_step_hip", *step_args(0, 2048, 128))  # B == 0: no-op
    # Later stages are checked before the first launch too (no GPU here: a
    # launch would fail with a HIP error instead of these messages), so a
    # refused step leaves the conv caches and x_n history untouched.
    with pytest.raises(GdnError, match="decode: dv=16"):
        abi.call("gdn_layer_decode_step_hip", *step_args(4, 2048, 16))
    misaligned = step_args(4, 2048, 128)
    misaligned[11] = FAKE + 4  # S_in
    with pytest.raises(GdnError, match="decode: q/k/S/o need 16-byte"):
        abi.call("gdn_layer_decode_step_hip", *misaligned)


def test_binding_module_api_matches_reference():
    """Module names, attrs and signatures of the reference's pybind modules."""
    exts = compile_kernels()
    assert set(exts) == {"rmsnorm", "proj", "prefill", "decode"}
    pf = exts["prefill"]
    assert (pf.H_DIM, pf.K_DIM, pf.V_DIM, pf.C_DIM) == (16, 128, 256, 64)
    sig = pf.prefill.__doc__.split("(", 1)[1].split(")", 1)[0]
    names = [a.split(":")[0].strip() for a in sig.split(",")]
    # the reference's ten positional arguments, then keyword-only additions
    assert names[:10] == ["q", "k", "v", "A_log", "a", "dt_bias", "b_logits", "mask", "state_in", "scale"]
    assert names[10:] == ["*", "token_major"]
    for mod in ("decode", "rmsnorm", "proj"):
        assert hasattr(exts[mod], "forward")


def test_binding_rejects_cpu_tensors():
    exts = compile_kernels()
    q = torch.zeros(1, 2, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        exts["prefill"].prefill(q, q, q, torch.zeros(2), torch.zeros(1, 2, 64, dtype=torch.bfloat16), 0.0,
                                torch.zeros(1, 2, 64, dtype=torch.bfloat16), torch.ones(1, 64), torch.empty(0), 0.0)
    with pytest.raises(RuntimeError, match="must be >= 32"):
        exts["rmsnorm"].forward(torch.zeros(2, 8, dtype=torch.bfloat16), torch.ones(8, dtype=torch.bfloat16),
                                1e-6, 16, 1)
