"""The no-allocation prefill entry point (gdn_prefill_noalloc_hip) against
gdn_prefill_hip with a caller workspace, through the C ABI.

Both run the same kernels on the same inputs, so their outputs and final
states must be bit-identical.  Two calls in a row share the library's static
scratch buffer; the second is smaller, so leftovers of the first call must
not leak into it.  A shape beyond the buffer is refused before any launch.
"""

import pytest
import torch

from gdn_18646_amd import abi, synth
from gdn_18646_amd.abi import GdnError

pytestmark = pytest.mark.gpu


def _run(entry, g, B, H, T, dv, dev):
    out = torch.full((B, H, T, dv), float("nan"), dtype=torch.bfloat16, device=dev)
    S = torch.full((B, H, 128, dv), float("nan"), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    args = [g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(), g["A_log"].data_ptr(), g["a"].data_ptr(),
            float(g["dt_bias"]), g["b_logits"].data_ptr(), g["mask"].data_ptr(),
            g["state_in"].data_ptr() if g.get("state_in") is not None else None, 0.0, out.data_ptr(), S.data_ptr(),
            B, H, T, 128, dv]
    if entry == "gdn_prefill_hip":
        nbytes = abi.load().gdn_prefill_workspace_bytes(B, H, T, 128, dv)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        abi.call(entry, *args, ws.data_ptr(), nbytes, stream)
    else:
        abi.call(entry, *args, stream)
    torch.cuda.synchronize()
    return out.cpu(), S.cpu()


@pytest.mark.parametrize("shapes", [((1, 8192, 16, 128, False), (2, 300, 4, 64, True))])
def test_noalloc_matches_workspace_entry(dev, shapes):
    for B, T, H, dv, with_state in shapes:  # the second call is the smaller one
        print(f"noalloc case B={B} T={T} H={H} dv={dv} state={with_state}", flush=True)
        d = synth.prefill_inputs(B, T, H, 128, dv, seed=7, state=with_state)
        g = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}
        o_ref, S_ref = _run("gdn_prefill_hip", g, B, H, T, dv, dev)
        o_na, S_na = _run("gdn_prefill_noalloc_hip", g, B, H, T, dv, dev)
        assert torch.isfinite(o_na.float()).all() and torch.isfinite(S_na).all()
        assert torch.equal(o_na, o_ref), "no-allocation output differs from the workspace entry point"
        assert torch.equal(S_na, S_ref), "no-allocation final state differs from the workspace entry point"


def test_noalloc_refuses_oversized_shape(dev):
    with pytest.raises(GdnError, match="WORKSPACE"):
        abi.call("gdn_prefill_noalloc_hip", *([4096] * 5), 0.0, 4096, 4096, None, 0.0, 4096, 4096,
                 8, 16, 65536, 128, 128, None)


def test_noalloc_under_graph_capture(dev):
    """The no-allocation entry point captured in a HIP graph (its callers'
    case): three replays on new inputs copied into the captured tensors, with
    eager work between them, each bit-identical to gdn_prefill_hip on the same
    inputs (4 chunk groups: intra kernel, map pass, scan, output pass)."""
    B, H, T, dv = 1, 4, 1000, 128
    ins = [synth.prefill_inputs(B, T, H, 128, dv, seed=60 + i, state=True) for i in range(4)]
    keys = ("q", "k", "v", "a", "b_logits", "state_in")
    g = {k: (v.to(dev).clone() if torch.is_tensor(v) else v) for k, v in ins[0].items()}
    out = torch.empty(B, H, T, dv, dtype=torch.bfloat16, device=dev)
    S = torch.empty(B, H, 128, dv, dtype=torch.float32, device=dev)

    def call(stream):
        abi.call("gdn_prefill_noalloc_hip", g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(),
                 g["A_log"].data_ptr(), g["a"].data_ptr(), float(g["dt_bias"]), g["b_logits"].data_ptr(),
                 g["mask"].data_ptr(), g["state_in"].data_ptr(), 0.0, out.data_ptr(), S.data_ptr(),
                 B, H, T, 128, dv, stream)

    call(torch.cuda.current_stream().cuda_stream)  # first call on the device: looks up the static buffer
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(torch.cuda.current_stream().cuda_stream)
    for d in ins[1:]:
        for k in keys:
            g[k].copy_(d[k].to(dev))
        graph.replay()
        torch.cuda.synchronize()
        got_o, got_S = out.cpu(), S.cpu()
        ref_o, ref_S = _run("gdn_prefill_hip", g, B, H, T, dv, dev)
        assert torch.equal(got_o, ref_o) and torch.equal(got_S, ref_S)
        _ = torch.randn(1 << 20, device=dev).sum()  # unrelated eager work between replays
