"""GDN layer on the MI355X kernels — drop-in for the reference's gdn_layer.py.

Same module constants, weight dict, decode-state dict and ``forward`` /
``decode`` signatures as the reference (gdn_layer.py:24-40, 79-102, 206-316);
the architecture is read from the weight shapes, so the reference's shape
(H=16, DK=128, DV=256) and the brief's layer config (DV=128) both run.

Pipeline per call (all GPU, one stream):

  forward  RMSNorm kernel -> one fused q/k/v/a/b in-projection GEMM with the
           conv + SiLU epilogue writing the prefill kernel's head-major layout
           (and, on request, the conv cache for decode) -> chunked prefill
           (output written token-major) -> W_o GEMM.  No .item() host sync: dt_bias is read once at
           construction (call ``refresh()`` after changing the weights).
  decode   one host call per step.  B <= 16: the fused RMSNorm + q/k/v/a/b
           projection + conv step kernel, the decode kernel (state update in
           place when asked) and the W_o projection kernel.  Larger batches:
           RMSNorm kernel (+ x_n history) -> tiled
           in-projection with the conv step in its epilogue -> decode kernel
           -> tiled W_o projection.  Shapes outside both: RMSNorm kernel ->
           xn W^T GEMM -> decode conv step -> decode kernel -> W_o GEMM.

The baseline (pure PyTorch) layer of the reference is the oracle's
``oracle.layer_ref.GDNLayerBaseline``; it is test infrastructure, not shipped.
"""

import torch

from . import compile_kernels

# Reference defaults (gdn_layer.py:24-28).
D = 2048
H = 16
DK = 128
DV = 256
CONV_K = 4


def dims(weights):
    """(D, H, DK, DV, CONV_K) from a weight dict's shapes."""
    Hh = weights['A_log'].numel()
    return (weights['W_q'].shape[1], Hh, weights['W_q'].shape[0] // Hh, weights['W_v'].shape[0] // Hh,
            weights['conv_q'].shape[1])


def _zero_decode_state(weights, B, device=None):
    """Zeroed decode cache with the reference's keys (gdn_layer.py:31-40)."""
    Dd, Hh, dk, dv, ck = dims(weights)
    device = device or weights['norm_gamma'].device
    bf = torch.bfloat16
    return dict(
        recurrent=torch.zeros(B, Hh, dk, dv, dtype=torch.float32, device=device),
        conv_q=torch.zeros(B, Hh * dk, ck - 1, dtype=bf, device=device),
        conv_k=torch.zeros(B, Hh * dk, ck - 1, dtype=bf, device=device),
        conv_v=torch.zeros(B, Hh * dv, ck - 1, dtype=bf, device=device),
        xn=torch.zeros(B, ck - 1, Dd, dtype=bf, device=device),
    )


def _dt_bias_for_decode(dt_bias, H_=None):
    """Per-head dt_bias for the decode kernel (gdn_layer.py:72-76)."""
    if dt_bias.numel() == 1:
        return dt_bias.reshape(1).expand(H_ or H).contiguous()
    return dt_bias.contiguous()


def make_weights(device="cuda", *, D=D, H=H, DK=DK, DV=DV, CONV_K=CONV_K, std=None, generator=None):
    """Random weight dict (gdn_layer.py:79-102).

    Default initialisation follows the reference (fan-in scaled normals);
    ``std`` instead draws every projection and conv weight from N(0, std)
    (the brief's layer config uses std 0.02).  ``generator`` makes it
    reproducible (CPU generator; tensors are moved to ``device``).
    """
    def rnd(*shape, scale):
        return (torch.randn(*shape, generator=generator) * scale).to(torch.bfloat16).to(device)

    def proj(rows, cols, extra=1.0):
        return rnd(rows, cols, scale=std if std is not None else cols ** -0.5 * extra)

    def conv(rows):
        return rnd(rows, CONV_K, scale=std if std is not None else CONV_K ** -0.5)

    return dict(
        norm_gamma=torch.ones(D, dtype=torch.bfloat16, device=device),
        W_q=proj(H * DK, D, DK ** -0.5), conv_q=conv(H * DK),
        W_k=proj(H * DK, D, DK ** -0.5), conv_k=conv(H * DK),
        W_v=proj(H * DV, D, DK ** -0.5), conv_v=conv(H * DV),
        W_a=proj(H, D), W_b=proj(H, D),
        A_log=torch.zeros(H, dtype=torch.float32, device=device),
        dt_bias=torch.tensor(0.0, dtype=torch.float32, device=device),
        W_o=proj(D, H * DV),
    )


class GDNLayerCustom:
    """Forward/decode of one GDN layer on the HIP kernels (gdn_layer.py:206-316)."""

    def __init__(self, weights, exts=None):
        self.w = weights
        self.exts = exts if exts is not None else compile_kernels()
        self._layer = _layer_module(self.exts)
        self.D, self.H, self.DK, self.DV, self.CK = dims(weights)
        self.scale = self.DK ** -0.5
        self.chunk = int(self.exts['prefill'].C_DIM)
        self._scratch = {}
        self.refresh()

    def refresh(self):
        """Re-derive the fused weights and gate constants from self.w."""
        w = self.w
        self.W_qkvab = torch.cat([w['W_q'], w['W_k'], w['W_v'], w['W_a'], w['W_b']], 0).contiguous()
        self.conv_qkv = torch.cat([w['conv_q'], w['conv_k'], w['conv_v']], 0).contiguous()
        self.A_log = w['A_log'].float().contiguous()
        dtb = w['dt_bias'].float()
        self.dt_bias_scalar = float(dtb.reshape(-1)[0].item()) if dtb.numel() == 1 else None
        self.dt_bias_vec = _dt_bias_for_decode(dtb, self.H).float().contiguous()
        self.W_o = w['W_o'].contiguous()
        self.gamma = w['norm_gamma'].contiguous()
        # Fused decode step: skinny projections for B <= 16, MFMA tiles
        # above.
        Hk, Hv = self.H * self.DK, self.H * self.DV
        self.fused_decode = (self.D % 32 == 0 and self.D <= 4096 and Hv % 32 == 0
                             and Hv <= 4096 and 1 <= self.CK <= 4)
        self.tiled_decode = (self.D % 64 == 0 and self.D <= 16384 and Hk % 64 == 0 and Hv % 64 == 0
                             and 1 <= self.CK <= 4)

    def init_decode_state(self, B, device=None):
        return _zero_decode_state(self.w, B, device=device)

    def _decode_scratch(self, B, device):
        """Intermediates of the fused decode step, kept across steps, one set per
        (B, device, stream): decode steps on different streams (and a graph
        captured on its capture stream, replayed beside eager steps) do not
        share them.  Steps of one batch size issued on one stream run in order."""
        key = (B, str(device), torch.cuda.current_stream(device).cuda_stream)
        buf = self._scratch.get(key)
        if buf is None:
            bf = dict(dtype=torch.bfloat16, device=device)
            Hh, dk, dv = self.H, self.DK, self.DV
            buf = (torch.empty(B, Hh, dk, **bf), torch.empty(B, Hh, dk, **bf), torch.empty(B, Hh, dv, **bf),
                   torch.empty(B, Hh, **bf), torch.empty(B, Hh, **bf),
                   torch.empty(B, Hh, dv, dtype=torch.float32, device=device))
            self._scratch[key] = buf
        return buf

    def _rmsnorm(self, x2d):
        return self.exts['rmsnorm'].forward(x2d.contiguous(), self.w['norm_gamma'], 1e-6, 256, 2)

    def _out_proj(self, o2d):
        """y = o W_o^T for o [M, H dv] bf16 (library GEMM).  Rows past the last
        multiple of 256 go in a second call: the library's 256-row tiles
        would otherwise add a whole round of tiles for them (M = 24,674:
        230 -> 169 us, the same numbers)."""
        M = o2d.shape[0]
        Mm = M - M % 256
        if Mm == 0 or Mm == M:
            return o2d @ self.W_o.T
        y = torch.empty(M, self.W_o.shape[0], dtype=o2d.dtype, device=o2d.device)
        torch.matmul(o2d[:Mm], self.W_o.T, out=y[:Mm])
        torch.matmul(o2d[Mm:], self.W_o.T, out=y[Mm:])
        return y

    @torch.no_grad()
    def forward(self, x, mask=None, return_state=False, state=None, cu_seqlens=None):
        """x [B, T, D] bf16 -> y [B, T, D] bf16.

        mask [B, T] fp32 (1 keep, 0 masked; default all ones).  With
        ``return_state`` also returns the decode-state dict after the last
        token (recurrent state and conv caches), so decode can continue the
        sequence.  ``state`` (optional) continues from an earlier state
        (initial recurrent state and conv caches).

        ``cu_seqlens`` [N + 1] (host offsets: a list or CPU tensor) makes x
        N packed sequences, x [1, T_total, D] (or [T_total, D]); every
        sequence is its own prefill (its conv and state start from zero, or
        from ``state``'s entry i), mask is [T_total] or [1, T_total], and the
        returned state has one entry per sequence (recurrent [N, H, dk, dv],
        conv caches [N, H d, K - 1], xn [N, K - 1, D]), which decode continues
        as a batch of N.
        """
        if self.dt_bias_scalar is None:
            raise ValueError("prefill takes a scalar dt_bias (as the reference kernel)")
        if cu_seqlens is not None:
            return self._forward_packed(x, cu_seqlens, mask, return_state, state)
        B, T, _ = x.shape
        Dd, Hh, dk, dv = self.D, self.H, self.DK, self.DV
        if mask is None:  # empty = every token kept (no fill kernel)
            mask = torch.empty(0, dtype=torch.float32, device=x.device)
        xn = self._rmsnorm(x.reshape(B * T, Dd)).reshape(B, T, Dd)
        st = state or {}
        outs = self._layer.in_proj(xn, self.W_qkvab, self.conv_qkv, Hh, dk, dv,
                                   st.get('conv_q'), st.get('conv_k'), st.get('conv_v'), bool(return_state))
        q, k, v, a, b = outs[:5]
        s_in = st.get('recurrent')
        if s_in is None:
            s_in = torch.empty(0, dtype=torch.float32, device=x.device)
        # token-major output [B, T, H, dv]: feeds W_o without a transpose copy
        o, S = self.exts['prefill'].prefill(q, k, v, self.A_log, a, self.dt_bias_scalar, b, mask.contiguous(),
                                            s_in, self.scale, token_major=True)
        y = self._out_proj(o.reshape(B * T, Hh * dv)).reshape(B, T, self.D)
        if not return_state:
            return y
        # x_n history: the last nc normalised tokens, the given state's (zeros
        # without one) in front when T < nc.  Only those rows are copied.
        nc = self.CK - 1
        if T >= nc:
            xn_hist = xn[:, T - nc:]
        else:
            prev = st.get('xn')
            if prev is None:
                prev = torch.zeros(B, nc, Dd, dtype=x.dtype, device=x.device)
            xn_hist = torch.cat([prev[:, T:], xn], 1)
        return y, dict(recurrent=S, conv_q=outs[5], conv_k=outs[6], conv_v=outs[7], xn=xn_hist.contiguous())

    def _forward_packed(self, x, cu_seqlens, mask, return_state, state):
        Dd, Hh, dk, dv = self.D, self.H, self.DK, self.DV
        cu = torch.as_tensor(cu_seqlens, dtype=torch.int32).cpu().contiguous()
        N = cu.numel() - 1
        Tt = x.shape[-2]
        if x.shape[-1] != Dd or x.numel() != Tt * Dd:
            raise ValueError(f"packed x must be [1, T_total, D] or [T_total, D], got {tuple(x.shape)}")
        xn = self._rmsnorm(x.reshape(Tt, Dd))
        st = state or {}
        outs = self._layer.in_proj_varlen(xn, self.W_qkvab, self.conv_qkv, Hh, dk, dv, cu, st.get('conv_q'),
                                          st.get('conv_k'), st.get('conv_v'), bool(return_state))
        q, k, v, a, b = outs[:5]
        s_in = st.get('recurrent')
        if s_in is None:
            s_in = torch.empty(0, dtype=torch.float32, device=x.device)
        m = None if mask is None else mask.reshape(-1).float().contiguous()
        # token-major output [1, T_total, H, dv]: feeds W_o without a transpose copy
        o, S = self.exts['prefill'].prefill_varlen(q, k, v, self.A_log, a, self.dt_bias_scalar, b, cu, s_in,
                                                   self.scale, mask=m, token_major=True)
        y = self._out_proj(o.reshape(Tt, Hh * dv)).reshape(x.shape)
        if not return_state:
            return y
        # x_n history: the last K - 1 tokens of each sequence, earlier ones from
        # the given state (zeros without one) where the sequence is shorter.
        # Only the wanted rows are gathered: from x_n, or from the given state
        # (zeros without one) for the positions before a sequence's start.
        nc = self.CK - 1
        from_x, from_prev = ([], []), ([], [])  # (history row, source row)
        for i in range(N):
            lo, hi = int(cu[i]), int(cu[i + 1])
            for j in range(nc):
                t = hi - nc + j  # packed token index wanted
                dst = from_x if t >= lo else from_prev
                dst[0].append(i * nc + j)
                dst[1].append(t if t >= lo else i * nc + nc - (lo - t))
        dev = x.device
        hist = torch.empty(N * nc, Dd, dtype=xn.dtype, device=dev)
        if from_x[0]:
            rows = torch.tensor(from_x[0], dtype=torch.long, device=dev)
            hist.index_copy_(0, rows, xn.index_select(0, torch.tensor(from_x[1], dtype=torch.long, device=dev)))
        if from_prev[0]:
            rows = torch.tensor(from_prev[0], dtype=torch.long, device=dev)
            prev = st.get('xn')
            if prev is None:
                hist.index_fill_(0, rows, 0)
            else:
                src = prev.reshape(N * nc, Dd).index_select(0, torch.tensor(from_prev[1], dtype=torch.long, device=dev))
                hist.index_copy_(0, rows, src)
        return y, dict(recurrent=S, conv_q=outs[5], conv_k=outs[6], conv_v=outs[7], xn=hist.reshape(N, nc, Dd))

    @torch.no_grad()
    def decode(self, x, state=None, inplace=False):
        """One token: x [B, 1, D] -> (y [B, 1, D], new state dict).

        The conv caches of the state dict hold the last CONV_K-1 projected
        tokens (the reference baseline's decode semantics).  With
        ``inplace=True`` the state tensors are updated in place and the same
        dict is returned (no allocation of a new 4-D state per step).
        The fused step keeps its q/k/v/a/b/o intermediates per (batch size,
        device, stream), so concurrent decodes of one layer must run on
        different streams (or different batch sizes).
        """
        B, T, _ = x.shape
        assert T == 1, f"decode expects T=1, got T={T}"
        Dd, Hh, dk, dv = self.D, self.H, self.DK, self.DV
        if state is None:
            state = self.init_decode_state(B, device=x.device)
        if inplace:
            cq, ck, cv, S_out = state['conv_q'], state['conv_k'], state['conv_v'], state['recurrent']
        else:
            cq, ck, cv = (state[n].clone() for n in ('conv_q', 'conv_k', 'conv_v'))
            S_out = torch.empty_like(state['recurrent'])
        # the fused step: skinny projections up to 16 sequences, tiles above
        # (config 5: 37 us at B=32, 123 at B=256, against 76 and 139 for the
        # library-GEMM path)
        fused = (self.fused_decode and B <= 16) or (self.tiled_decode and 16 < B <= 65535)
        if fused:
            # The whole step in one host call: RMSNorm + projections + conv
            # step + x_n history, the recurrence, the output projection.
            xn_hist = state['xn'] if inplace else state['xn'].clone()
            q, k, v, a, b, o = self._decode_scratch(B, x.device)
            y = torch.empty(B, 1, Dd, dtype=torch.bfloat16, device=x.device)
            self._layer.decode_step(x.reshape(B, Dd).contiguous(), self.gamma, 1e-6, self.W_qkvab, self.conv_qkv,
                                    cq, ck, cv, xn_hist, self.A_log, self.dt_bias_vec, state['recurrent'], S_out,
                                    self.scale, self.W_o, q, k, v, a, b, o, y.view(B, Dd), Hh, dk, dv)
            if inplace:
                return y, state
            return y, dict(recurrent=S_out, conv_q=cq, conv_k=ck, conv_v=cv, xn=xn_hist)
        # Shapes the fused step does not take: library GEMMs
        # around the conv-step and decode kernels.
        xn = self._rmsnorm(x.reshape(B, Dd))
        P = xn @ self.W_qkvab.T
        # the conv-step launch also shifts the x_n history (in place: the
        # state's own tensor, so a captured step stays valid, or a copy)
        xn_hist = state['xn'] if inplace else state['xn'].clone()
        q, k, v, a, b = self._layer.decode_conv_step(P, self.conv_qkv, cq, ck, cv, Hh, dk, dv, xn, xn_hist)
        o = torch.empty(B, Hh, dv, dtype=torch.float32, device=x.device)
        self.exts['decode'].forward(q, k, v, a, b, self.A_log, self.dt_bias_vec, state['recurrent'], self.scale,
                                    o, S_out)
        y = o.to(x.dtype).reshape(B, 1, Hh * dv) @ self.W_o.T
        if inplace:
            return y, state
        return y, dict(recurrent=S_out, conv_q=cq, conv_k=ck, conv_v=cv, xn=xn_hist.contiguous())

    def capture_decode(self, state, warmup=2):
        """One in-place decode step of this layer captured as a HIP graph.

        Returns ``step(x) -> y``: copies x [B, 1, D] into the graph's input
        buffer, replays the graph and returns its output buffer (y [B, 1, D],
        overwritten by the next call).  ``state`` (a decode-state dict, e.g.
        from ``forward(..., return_state=True)``) is updated in place by
        every call, exactly as ``decode(x, state, inplace=True)``.  The decode
        step is a chain of small launches, so replaying it as one graph
        removes the per-launch host overhead.  The warm-up steps run on copies
        of the state values, which are then restored.
        """
        B = state['recurrent'].shape[0]
        dev = state['recurrent'].device
        x_static = torch.zeros(B, 1, self.D, dtype=torch.bfloat16, device=dev)
        saved = {k: v.clone() for k, v in state.items()}
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.decode(x_static, state, inplace=True)
        torch.cuda.current_stream(dev).wait_stream(side)
        for k, v in state.items():
            v.copy_(saved[k])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_static, _ = self.decode(x_static, state, inplace=True)
        del saved

        def step(x):
            x_static.copy_(x)
            graph.replay()
            return y_static

        step.graph = graph
        return step


def _layer_module(exts):
    """The binding's layer submodule (kept beside the four reference modules)."""
    from . import native_extension
    return native_extension().layer
