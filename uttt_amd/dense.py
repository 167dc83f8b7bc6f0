"""uTTT-Dense fast-weight path on the gfx950 grouped kernels.

uTTT-Dense keeps one SwiGLU fast weight per head (w0, w2 [b, H, d_h, d],
w1 [b, H, d, d_h]) shared by all layers.  Each head is one batch of the
grouped kernels with a single expert (group_sizes = [[N]]), so the read is
the grouped APPLY and a layer's update the grouped UPDATE.  Reference:
uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py (D:):

  apply_fast_weights   _apply_fast_weights  D:241-268 (the output; the
                       reference's intermediate views are not returned)
  compute_update       compute_update       D:333-449 from the preprocessed
                       k, v, lr (fp32 raw update, stored bf16 as under autocast)
  SharedFastWeights    the shared bank of D:1801-1863: read() per layer and
                       chunk, write() = _aggregate_memory_update D:1302-1386 +
                       _apply_shared_update D:1109-1240

Reads of more than DECODE_TOKENS tokens with small heads (d in {64, 96, 128,
192, 256}, d_h a multiple of 32 up to 512) run the fused read of
csrc/dense_read.hip on the [b, l, H*d] activations directly; other shapes
split the heads (csrc/dense_heads.hip) and run the grouped APPLY.

SharedFastWeights keeps its state in the kernels' layout -- fast W0_W2
[b*H, 1, 2 d_h, d] and W1 [b*H, 1, d, d_h] in bf16 with fp32 masters -- so a
chunk needs no concatenation or copy of the weights.  Its write batches the L
layers: their tokens are concatenated per head into one UPDATE call, whose
fp32 accumulation gives sum_l dW_l (the reference adds the layers' bf16
updates in fp32); the mean reduce is folded into the step size.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from .decode import moe_decode_read
from .lact_moe_triton import _grouped as G

# Reads of at most this many tokens (generation) stream the weights with the
# decode kernels (csrc/decode_read.hip, one "expert" per head, gate 1): the
# grouped GEMM would spend a 256-token tile on them.  Same rounding points:
# bf16 hidden, bf16 output (the gate-1 merge is exact).
DECODE_TOKENS = 8


def _bf16_rows(x):
    x = x.to(torch.bfloat16)
    return x if x.is_contiguous() else x.contiguous()


def _gather_heads(ks, vs, lrs, H):
    """One launch (csrc/dense_heads.hip): the layers' k [b, l, H*d] (and v,
    and lr [b, l, 3] or [b, l, H*3]) -> per head with the layers' tokens
    concatenated: kh, vh [b*H, L*l, d] bf16 and lr0/1/2 [b*H, L*l] fp32
    (D:370-398 per layer, the layers batched as the aggregate write needs)."""
    ks = [_bf16_rows(k) for k in ks]
    b, l, hd = ks[0].shape
    n = len(ks)
    for k in ks:
        assert k.shape == (b, l, hd), "every layer's k, v: [b, l, H*d] of one shape"
    d = hd // H
    dev = ks[0].device
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])
    kh = torch.empty((b * H, n * l, d), dtype=torch.bfloat16, device=dev)
    vh = lr3 = None
    vp = lp = None
    if vs is not None:
        vs = [_bf16_rows(v) for v in vs]
        for v in vs:
            assert v.shape == (b, l, hd), "every layer's k, v: [b, l, H*d] of one shape"
        vh = torch.empty_like(kh)
        vp = arr(vs)
    per_head, code = 0, L.F32
    if lrs is not None:
        lrs = [lr.contiguous() for lr in lrs]
        code = L.dtype_code(lrs[0].dtype)
        per_head = int(lrs[0].shape[2] != 3)
        for lr in lrs:
            assert lr.dtype == lrs[0].dtype and lr.shape == (b, l, 3 * H if per_head else 3)
        lr3 = [torch.empty((b * H, n * l), dtype=torch.float32, device=dev) for _ in range(3)]
        lp = arr(lrs)
    L.call("uttt_dense_gather_heads", arr(ks), vp, lp, code, per_head, n, b, l, H, d,
           L.ptr(kh), L.ptr(vh), *(L.ptr(x) for x in (lr3 or [None] * 3)), L.stream_of(kh))
    return kh, vh, lr3


def _heads(x, H):
    """D:251: [b, l, H*d] -> contiguous [b*H, l, d] bf16."""
    return _gather_heads([x], None, None, H)[0]


def _unheads(y, b, H):
    """D:261: [b*H, l, d] bf16 -> [b, l, H*d]."""
    bh, l, d = y.shape
    out = torch.empty((b, l, H * d), dtype=torch.bfloat16, device=y.device)
    L.call("uttt_dense_scatter_heads", L.ptr(y.contiguous()), b, l, H, d, L.ptr(out),
           L.stream_of(y))
    return out


_GS = {}


def _gs(B, N, device):
    """group_sizes [[N]] * B (one expert per head), kept per shape and device:
    read-only for the kernels, so one tensor serves every call."""
    key = (B, N, str(device))
    gs = _GS.get(key)
    if gs is None:
        gs = _GS[key] = torch.full((B, 1), N, dtype=torch.int32, device=device)
    return gs


def apply_fast_weights(x, w0, w1, w2):
    """D:241-268.  x [b, l, H*d] -> out [b, l, H*d] (bf16)."""
    b, H, dh, d = w0.shape
    W02 = torch.cat([w0, w2], dim=2).to(torch.bfloat16).reshape(b * H, 1, 2 * dh, d).contiguous()
    W1 = w1.to(torch.bfloat16).reshape(b * H, 1, d, dh).contiguous()
    return _read(x, W02, W1, b, H)


def _read(x, W02, W1, b, H):
    L.require_device(x)
    d, dh = W1.shape[-2], W1.shape[-1]
    assert x.dim() == 3 and x.shape[2] == H * d, "x: [b, l, H*d]"
    if x.shape[1] > DECODE_TOKENS and L.lib().uttt_dense_read_supported(d, dh):
        # fused (csrc/dense_read.hip): x and out stay in the [b, l, H*d] layout
        xb = _bf16_rows(x)
        out = torch.empty_like(xb)
        L.call("uttt_dense_read", L.ptr(xb), b, xb.shape[1], H, d, L.ptr(W02), L.ptr(W1), dh,
               L.ptr(out), L.stream_of(xb))
        return out
    xh = _heads(x, H)
    if xh.shape[1] <= DECODE_TOKENS:
        ones = torch.ones((b * H, 1, xh.shape[1]), dtype=torch.float32, device=x.device)
        return _unheads(moe_decode_read(xh, W02, W1, ones.to(torch.uint8), ones, 1), b, H)
    gs = _gs(b * H, xh.shape[1], x.device)
    hid = G.gate_up(W02, xh, gs, token_major=True)
    return _unheads(G.gemm_nt(W1, hid, gs), b, H)


def _pack(W02, W1, packed=None):
    """The fragment-ordered copy of the weights that uttt_dense_read_packed
    reads (csrc/dense_read.hip), or None where the fused read does not apply."""
    BH, d, dh = W02.shape[0], W1.shape[-2], W1.shape[-1]
    if not L.lib().uttt_dense_read_supported(d, dh):
        return None
    if packed is None:
        packed = torch.empty(BH * 3 * dh * d, dtype=torch.bfloat16, device=W02.device)
    L.call("uttt_dense_pack_weights", L.ptr(W02), L.ptr(W1), BH, d, dh, L.ptr(packed),
           L.stream_of(W02))
    return packed


def _read_packed(x, packed, W02, W1, b, H):
    """_read with the weights' packed copy for the fused read."""
    d, dh = W1.shape[-2], W1.shape[-1]
    if packed is None or x.shape[1] <= DECODE_TOKENS:
        return _read(x, W02, W1, b, H)
    L.require_device(x)
    assert x.dim() == 3 and x.shape[2] == H * d, "x: [b, l, H*d]"
    xb = _bf16_rows(x)
    out = torch.empty_like(xb)
    L.call("uttt_dense_read_packed", L.ptr(xb), b, xb.shape[1], H, d, L.ptr(packed), dh,
           L.ptr(out), L.stream_of(xb))
    return out


def _pack_update(W02, W1, packed=None):
    """The fragment-ordered copy of the weights that uttt_dense_update_stage1
    reads (csrc/dense_update.hip)."""
    BH, d, dh = W02.shape[0], W1.shape[-2], W1.shape[-1]
    if packed is None:
        packed = torch.empty(BH * 3 * dh * d, dtype=torch.bfloat16, device=W02.device)
    L.call("uttt_dense_pack_update_weights", L.ptr(W02), L.ptr(W1), BH, d, dh, L.ptr(packed),
           L.stream_of(W02))
    return packed


def _update_stage1(W02, W1, kh, vh, lr3, gs, upacked=None):
    """(DY0_DY2 [BH, N, 2I], Hid [BH, N, I]) bf16 token-major: the fused
    kernel for small heads, else the grouped stage 1 (E = 1)."""
    d, dh = W1.shape[-2], W1.shape[-1]
    if not L.lib().uttt_dense_update_supported(d, dh):
        return G.update_stage1(W02, W1, kh, vh, *(lr3 or (None,) * 3), gs, token_major=True)
    upacked = _pack_update(W02, W1, upacked)
    BH, N = kh.shape[0], kh.shape[1]
    dy = torch.empty((BH, N, 2 * dh), dtype=torch.bfloat16, device=kh.device)
    hl = torch.empty((BH, N, dh), dtype=torch.bfloat16, device=kh.device)
    L.call("uttt_dense_update_stage1", L.ptr(kh), L.ptr(vh), *(L.ptr(x) for x in (lr3 or (None,) * 3)),
           BH, N, d, dh, L.ptr(upacked), L.ptr(dy), L.ptr(hl), L.stream_of(kh))
    return dy, hl


def _layered(ks, vs, lrs, H, d, dh):
    """The layers' own k, v (bf16 [b, l, H*d], 16-byte aligned) and lr for
    the layered UPDATE (no per-head copy), or None where it does not apply:
    the fused stage 1's head sizes, l a multiple of 64, at most 64 layers."""
    n = len(ks)
    if not (1 <= n <= 64 and vs is not None and len(vs) == n
            and L.lib().uttt_dense_update_supported(d, dh)):
        return None
    ks = [_bf16_rows(k) for k in ks]
    vs = [_bf16_rows(v) for v in vs]
    b, l, hd = ks[0].shape
    if l % 64 or hd != H * d or any(t.shape != (b, l, hd) for t in ks + vs):
        return None
    if any(t.data_ptr() % 16 for t in ks + vs):
        return None
    if lrs is not None:
        lrs = [lr.contiguous() for lr in lrs]
        if any(lr.dtype != lrs[0].dtype or lr.shape not in ((b, l, 3), (b, l, 3 * H))
               or lr.shape != lrs[0].shape for lr in lrs):
            return None
    return ks, vs, lrs, b, l


def _update_layered(W02, W1, ks, vs, lrs, b, l, H, upacked):
    """The UPDATE of several layers straight from each layer's own k, v, lr
    (uttt_dense_update_stage1_layers, uttt_dense_wgrad_pair_layers): the same
    products as the per-head copy path, the weight gradients split into one K
    run per layer."""
    d, dh = W1.shape[-2], W1.shape[-1]
    n, BH, N = len(ks), b * H, len(ks) * l
    dev = ks[0].device
    upacked = _pack_update(W02, W1, upacked)
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])
    dy = torch.empty((BH, N, 2 * dh), dtype=torch.bfloat16, device=dev)
    hl = torch.empty((BH, N, dh), dtype=torch.bfloat16, device=dev)
    per_head = int(lrs is not None and lrs[0].shape[2] != 3)
    code = L.dtype_code(lrs[0].dtype) if lrs is not None else L.F32
    st = L.stream_of(dy)
    L.call("uttt_dense_update_stage1_layers", arr(ks), arr(vs), arr(lrs) if lrs else None, code,
           per_head, n, b, l, H, d, dh, L.ptr(upacked), L.ptr(dy), L.ptr(hl), st)
    dW02 = torch.empty((BH, 1, 2 * dh, d), dtype=torch.bfloat16, device=dev)
    dW1 = torch.empty((BH, 1, d, dh), dtype=torch.bfloat16, device=dev)
    nws = L.lib().uttt_dense_wgrad_pair_layers_workspace_bytes(n, b, H, dh, d)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    L.call("uttt_dense_wgrad_pair_layers", L.ptr(dy), arr(ks), L.ptr(hl), arr(vs), n, b, l, H,
           dh, d, L.ptr(dW02), L.ptr(dW1), L.ptr(ws), nws, st)
    return dW02, dW1


def _update(W02, W1, ks, vs, lrs, b, H, upacked=None):
    """The UPDATE of several layers' tokens at once: per head the tokens of
    all layers concatenated.  Returns bf16 (dW0_W2, dW1).  upacked: a buffer
    of BH * 3 * d_h * d bf16 for the fused stage 1's weight copy.  Where the
    fused stage 1 applies and each layer's l is a multiple of 64, the kernels
    read every layer's own k, v and lr (no per-head copy)."""
    lay = _layered(ks, vs, lrs, H, W1.shape[-2], W1.shape[-1])
    if lay is not None:
        ks_, vs_, lrs_, b_, l_ = lay
        assert b_ == b
        return _update_layered(W02, W1, ks_, vs_, lrs_, b, l_, H, upacked)
    kh, vh, lr3 = _gather_heads(ks, vs, lrs, H)
    gs = _gs(b * H, kh.shape[1], kh.device)
    dy, hl = _update_stage1(W02, W1, kh, vh, lr3, gs, upacked)
    return G.wgrad_pair(dy, kh, hl, vh, gs)


def compute_update(k, v, lr, fastw):
    """D:333-449 from the preprocessed k, v [b, l, H*d] and lr [b, l, 3] or
    [b, l, H*3]: (dw0 [b,H,d_h,d], dw1 [b,H,d,d_h], dw2) in fp32."""
    w0, w1, w2 = fastw
    b, H, dh, d = w0.shape
    L.require_device(k, v, lr, w0)
    W02 = torch.cat([w0, w2], dim=2).to(torch.bfloat16).reshape(b * H, 1, 2 * dh, d).contiguous()
    W1 = w1.to(torch.bfloat16).reshape(b * H, 1, d, dh).contiguous()
    dW02, dW1 = _update(W02, W1, [k], [v], [lr], b, H)
    dW02 = dW02.float().reshape(b, H, 2 * dh, d)
    return dW02[:, :, :dh], dW1.float().reshape(b, H, d, dh), dW02[:, :, dh:]


class SharedFastWeights:
    """The shared fast-weight bank of uTTT-Dense (D:1801-1863), aggregate
    schedule: read() every layer of a chunk with the chunk-start weights, then
    write() once from the mean (or sum) of the layers' updates, projected per
    d x d slice onto the old slice norms (_apply_shared_update, D:1109-1240),
    with the optional momentum (the buffer keeps the pre-Muon aggregate,
    D:1175-1185) and Muon (Newton-Schulz per d x d slice, D:1192-1203) of the
    shipped configs.

    w0, w2: [b, H, r*d, d]; w1: [b, H, d, r*d]; masters fp32 (default: the
    given weights in fp32).  The bank owns its weights: weights() returns
    copies and set_weights() replaces them (and drops the read's packed copy)."""

    def __init__(self, w0, w1, w2, r, masters=None, lr_scale=1.0, reduce="mean",
                 master_renorm=False, use_momentum=False, use_moun=False):
        b, H, dh, d = w0.shape
        if dh != r * d or tuple(w1.shape) != (b, H, d, r * d) or w2.shape != w0.shape:
            raise ValueError(f"invalid shared fast state shapes for r={r}")
        if reduce not in ("mean", "sum"):
            raise ValueError(f"`uttt_agg_reduce` must be 'mean' or 'sum', got {reduce!r}.")
        L.require_device(w0, w1, w2)
        self.b, self.H, self.d, self.dh, self.r = b, H, d, dh, r
        self.lr_scale, self.reduce, self.master_renorm = float(lr_scale), reduce, master_renorm
        self.use_momentum, self.use_moun = bool(use_momentum), bool(use_moun)
        self._spare02 = torch.empty((b * H, 1, 2 * dh, d), dtype=torch.bfloat16, device=w0.device)
        self._spare1 = torch.empty((b * H, 1, d, dh), dtype=torch.bfloat16, device=w0.device)
        # The read's fragment-ordered copy of W02/W1 (one extra pass over the
        # weights) pays off only when the same weights are read more than once:
        # it is rebuilt at a write that aggregated several layers (the next
        # chunk's reads are as many), else at the second read after a write.
        supported = L.lib().uttt_dense_read_supported(d, dh)
        self.P = (torch.empty(b * H * 3 * dh * d, dtype=torch.bfloat16, device=w0.device)
                  if supported else None)
        self._upacked = (torch.empty(b * H * 3 * dh * d, dtype=torch.bfloat16, device=w0.device)
                         if L.lib().uttt_dense_update_supported(d, dh) else None)
        self.set_weights((w0, w1, w2), masters)

    def set_weights(self, fastw, masters=None, momentum=None):
        """Load (w0, w1, w2) fast weights (and fp32 masters, default the fast
        weights in fp32; and the momentum buffers, default zero) into the
        bank's own storage (copies: the writes update it in place)."""
        b, H, dh, d = self.b, self.H, self.dh, self.d
        w0, w1, w2 = fastw
        m0, m1, m2 = masters if masters is not None else fastw
        self.M02 = torch.cat([m0, m2], dim=2).float().reshape(b * H, 1, 2 * dh, d).contiguous()
        self.M1 = m1.to(torch.float32, copy=True).reshape(b * H, 1, d, dh).contiguous()
        self.W02 = torch.cat([w0, w2], dim=2).to(torch.bfloat16).reshape(b * H, 1, 2 * dh, d).contiguous()
        self.W1 = w1.to(torch.bfloat16, copy=True).reshape(b * H, 1, d, dh).contiguous()
        if momentum is not None:
            o0, o1, o2 = momentum
            self.MOM02 = torch.cat([o0, o2], dim=2).float().reshape(b * H, 1, 2 * dh, d).contiguous()
            self.MOM1 = o1.to(torch.float32, copy=True).reshape(b * H, 1, d, dh).contiguous()
        else:
            self.MOM02 = torch.zeros_like(self.M02) if self.use_momentum else None
            self.MOM1 = torch.zeros_like(self.M1) if self.use_momentum else None
        self._reads, self._packed = 0, False

    def read(self, q):
        """One layer's read of a chunk: q [b, l, H*d] -> [b, l, H*d] bf16."""
        self._reads += 1
        if self.P is not None and not self._packed and self._reads >= 2:
            _pack(self.W02, self.W1, self.P)
            self._packed = True
        return _read_packed(q, self.P if self._packed else None, self.W02, self.W1, self.b,
                            self.H)

    def _coeff(self, momentum_coeffs):
        """The per-(batch, head) momentum coefficient: the mean of the layers'
        [b, 1, 1, 1] coefficients (D:1140-1146), repeated over the heads."""
        c = (momentum_coeffs if torch.is_tensor(momentum_coeffs)
             else torch.stack(list(momentum_coeffs), dim=0).mean(dim=0))
        c = c.reshape(-1).float()
        assert c.numel() == self.b, "momentum coefficients must hold one value per batch"
        return c.repeat_interleave(self.H).contiguous()

    def _steps_moun(self, g02, g1, scale):
        """bf16(NS5(slice) * scale) of every d x d slice (D:1192-1209): the
        w0 / w2 rows are 2r row blocks of d per (batch, head), the w1 slices
        r column blocks of d."""
        from .fast_weight_write import newton_schulz5

        B, d, r = self.b * self.H, self.d, self.r
        # every slice is orthogonalised on its own, so the w0 / w2 and the w1
        # slices go through one call (one launch where the slices are small)
        sl1 = g1.reshape(B, d, r, d).permute(0, 2, 1, 3).reshape(B * r, d, d)
        s = newton_schulz5(torch.cat([g02.reshape(B * 2 * r, d, d), sl1], dim=0), scale)
        s02 = s[:B * 2 * r].reshape(B, 1, 2 * r * d, d)
        s1 = s[B * 2 * r:].reshape(B, r, d, d).permute(0, 2, 1, 3)
        return s02, s1.reshape(B, 1, d, r * d).contiguous()

    def write(self, ks, vs, lrs, momentum_coeffs=None):
        """The chunk's aggregate write from every layer's preprocessed k, v
        [b, l, H*d] and lr ([b, l, 3] or [b, l, H*3]); momentum_coeffs: the
        layers' [b, 1, 1, 1] momentum coefficients (a list, averaged) or one
        tensor, used when the bank has momentum."""
        dW02, dW1 = _update(self.W02, self.W1, ks, vs, lrs, self.b, self.H, self._upacked)
        per_layer = 1.0 / (len(ks) if self.reduce == "mean" else 1)
        st = L.stream_of(dW02)
        nf = 0 if self.master_renorm else 1
        B, d, dh = self.b * self.H, self.d, self.dh
        use_mom = self.use_momentum and momentum_coeffs is not None
        g02, g1, gdt, scale = dW02, dW1, L.BF16, self.lr_scale * per_layer
        mom02 = mom1 = cb = None
        if use_mom or self.use_moun:
            # the aggregate itself (the mean of the layers' updates) in fp32
            g02 = dW02.float().mul_(per_layer)
            g1 = dW1.float().mul_(per_layer)
            gdt, scale = L.F32, self.lr_scale
        if use_mom:
            cb = self._coeff(momentum_coeffs)
            mom02, mom1 = self.MOM02, self.MOM1
        if self.use_moun:
            if use_mom:
                from .fast_weight_write import _momentum
                g02 = self.MOM02 = _momentum(g02, self.MOM02, cb)
                g1 = self.MOM1 = _momentum(g1, self.MOM1, cb)
                mom02 = mom1 = cb = None
            g02, g1 = self._steps_moun(g02, g1, self.lr_scale)
            gdt, scale = L.BF16, 1.0
        # W0_W2 rows are whole d x d slice rows; W1 rows hold r slices of d
        L.call("uttt_write_step", L.ptr(self.M02), L.ptr(self.W02), L.ptr(g02), gdt,
               L.ptr(mom02), L.ptr(cb), scale, B, 2 * dh, d, d, nf, int(self.master_renorm),
               L.ptr(self.M02), L.ptr(self._spare02), L.ptr(mom02), st)
        L.call("uttt_write_step", L.ptr(self.M1), L.ptr(self.W1), L.ptr(g1), gdt,
               L.ptr(mom1), L.ptr(cb), scale, B, d, dh, d, nf, int(self.master_renorm),
               L.ptr(self.M1), L.ptr(self._spare1), L.ptr(mom1), st)
        self.W02, self._spare02 = self._spare02, self.W02
        self.W1, self._spare1 = self._spare1, self.W1
        self._reads, self._packed = 0, False
        if self.P is not None and len(ks) > 1:
            _pack(self.W02, self.W1, self.P)
            self._packed = True

    def weights(self):
        """Copies of ((w0, w1, w2) bf16, (w0, w1, w2) fp32 masters) in the
        reference layout (the bank keeps its own storage)."""
        b, H, dh, d = self.b, self.H, self.dh, self.d

        def split(W02, W1):
            w02 = W02.reshape(b, H, 2 * dh, d)
            return (w02[:, :, :dh].clone(), W1.reshape(b, H, d, dh).clone(),
                    w02[:, :, dh:].clone())

        return split(self.W02, self.W1), split(self.M02, self.M1)

    def momentum(self):
        """Copies of the (w0, w1, w2) momentum buffers, or None."""
        if self.MOM02 is None:
            return None
        b, H, dh, d = self.b, self.H, self.dh, self.d
        m = self.MOM02.reshape(b, H, 2 * dh, d)
        return m[:, :, :dh].clone(), self.MOM1.reshape(b, H, d, dh).clone(), m[:, :, dh:].clone()
