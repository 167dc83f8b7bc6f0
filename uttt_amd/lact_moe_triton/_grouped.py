"""Launch helpers shared by the grouped fast-weight modules: thin wrappers
over the C-ABI of csrc/grouped_gemm.hip that allocate outputs with torch and
launch on torch's current stream.  No CPU path: CPU tensors raise.

Token-major intermediates ("_tok" suffix) are [B, N, rows] with rows
contiguous; the reference's kernel-level functions exchange [B, rows, N].
Every launch helper is registered as a torch.ops.uttt_hip op with a fake
implementation (uttt_amd._ops), so torch.compile traces it.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from uttt_amd import _lib as L  # absolute: the package also works mounted in the reference tree
from uttt_amd._ops import traced_op


def _check_bf16(*ts):
    for t in ts:
        assert t.dtype == torch.bfloat16, f"expected bf16, got {t.dtype}"
        assert t.is_contiguous(), "expected a contiguous tensor"


def group_sizes_i32(group_sizes: torch.Tensor) -> torch.Tensor:
    gs = group_sizes if group_sizes.dtype == torch.int32 else group_sizes.to(torch.int32)
    return gs.contiguous()


def _gate_up_fake(W0_W2, X, group_sizes, token_major):
    B, N, I = X.shape[0], X.shape[1], W0_W2.shape[2] // 2
    return X.new_empty((B, N, I) if token_major else (B, I, N))


@traced_op("grouped_gate_up", _gate_up_fake)
def gate_up(W0_W2: Tensor, X: Tensor, group_sizes: Tensor, token_major: bool) -> Tensor:
    """silu(w0 x) * (w2 x) per routed token: [B, N, I] (token_major) or [B, I, N]."""
    L.require_device(W0_W2, X, group_sizes)
    _check_bf16(W0_W2, X)
    B, E, I2, D = W0_W2.shape
    Bx, N, Dx = X.shape
    assert Bx == B and Dx == D, "X must be [B, N, D] with matching B, D"
    assert I2 % 2 == 0
    I = I2 // 2
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    shape = (B, N, I) if token_major else (B, I, N)
    H = torch.empty(shape, dtype=torch.bfloat16, device=X.device)
    L.call("uttt_grouped_gate_up", L.ptr(W0_W2), L.ptr(X), L.ptr(gs), B, E, I, D, N, L.ptr(H),
           int(token_major), L.stream_of(X))
    return H


def _gate_up_gather_fake(W0_W2, x, src_rows, group_sizes):
    return x.new_empty((x.shape[0], src_rows.shape[1], W0_W2.shape[2] // 2))


def gate_up_gathers(N: int, E: int) -> bool:
    """Whether gate_up_gather runs at N routed rows over E experts (the sizes
    that take the skinny tiles)."""
    return bool(L.lib().uttt_grouped_gate_up_gathers(int(N), int(E)))


@traced_op("grouped_gate_up_gather", _gate_up_gather_fake)
def gate_up_gather(W0_W2: Tensor, x: Tensor, src_rows: Tensor, group_sizes: Tensor) -> Tensor:
    """gate_up (token-major) of the routed rows x[b, src_rows[b, n]] of the
    unpermuted x [B, T, D]: [B, N, I] with N = src_rows.shape[1] (the inverse
    row map of route_tokens_map).  Where the sizes take the skinny tiles the
    kernel reads the rows through the index (no permuted copy); elsewhere the
    rows are gathered into a copy first (identical results)."""
    L.require_device(W0_W2, x, src_rows, group_sizes)
    _check_bf16(W0_W2, x)
    B, E, I2, D = W0_W2.shape
    Bx, T, Dx = x.shape
    assert Bx == B and Dx == D, "x must be [B, T, D] with matching B, D"
    assert src_rows.dtype == torch.int32 and src_rows.dim() == 2 and src_rows.shape[0] == B
    src_rows = src_rows.contiguous()
    N = src_rows.shape[1]
    if not gate_up_gathers(N, E):
        x_perm = torch.gather(x, 1, src_rows.long()[:, :, None].expand(B, N, D)).contiguous()
        return gate_up(W0_W2, x_perm, group_sizes, token_major=True)
    I = I2 // 2
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    H = torch.empty((B, N, I), dtype=torch.bfloat16, device=x.device)
    L.call("uttt_grouped_gate_up_gather", L.ptr(W0_W2), L.ptr(x), T, L.ptr(src_rows), N,
           L.ptr(gs), B, E, I, D, N, L.ptr(H), L.stream_of(x))
    return H


def _gemm_nt_fake(W, X_tok, group_sizes):
    return X_tok.new_empty((X_tok.shape[0], X_tok.shape[1], W.shape[2]))


@traced_op("grouped_gemm_nt", _gemm_nt_fake)
def gemm_nt(W: Tensor, X_tok: Tensor, group_sizes: Tensor) -> Tensor:
    """Y[b, n] = W[b, e(n)] @ X_tok[b, n]: W [B, E, M, K], X_tok [B, N, K] -> [B, N, M]."""
    L.require_device(W, X_tok, group_sizes)
    _check_bf16(W, X_tok)
    B, E, M, K = W.shape
    Bx, N, Kx = X_tok.shape
    assert Bx == B and Kx == K, "X must be [B, N, K] with matching B, K"
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    Y = torch.empty((B, N, M), dtype=torch.bfloat16, device=X_tok.device)
    L.call("uttt_grouped_gemm_nt", L.ptr(W), L.ptr(X_tok), L.ptr(gs), B, E, M, K, N, L.ptr(Y),
           L.stream_of(X_tok))
    return Y


def _gemm_tn_fake(W, X_tok, group_sizes):
    return X_tok.new_empty((X_tok.shape[0], X_tok.shape[1], W.shape[3]))


@traced_op("grouped_gemm_tn", _gemm_tn_fake)
def gemm_tn(W: Tensor, X_tok: Tensor, group_sizes: Tensor) -> Tensor:
    """Y[b, n] = W[b, e(n)]^T @ X_tok[b, n]: W [B, E, K, M], X_tok [B, N, K] -> [B, N, M]."""
    L.require_device(W, X_tok, group_sizes)
    _check_bf16(W, X_tok)
    B, E, K, M = W.shape
    Bx, N, Kx = X_tok.shape
    assert Bx == B and Kx == K, "X must be [B, N, K] with matching B, K"
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    Y = torch.empty((B, N, M), dtype=torch.bfloat16, device=X_tok.device)
    L.call("uttt_grouped_gemm_tn", L.ptr(W), L.ptr(X_tok), L.ptr(gs), B, E, M, K, N, L.ptr(Y),
           L.stream_of(X_tok))
    return Y


def update_stage1(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, token_major: bool,
                  save: bool = False):
    """See _update_stage1 (the registered op, which returns 0-element saves
    when save is False)."""
    out = _update_stage1(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, token_major, save)
    return out if save else out[:2]


def _update_stage1_fake(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes, token_major, save):
    B, N = K.shape[0], K.shape[1]
    I2 = W0_W2.shape[2]
    I = I2 // 2
    dy = K.new_empty((B, N, I2) if token_major else (B, I2, N))
    h = K.new_empty((B, N, I) if token_major else (B, I, N))
    ys = K.new_empty((B, N, I2) if save else (0,))
    dhs = K.new_empty((B, N, I) if save else (0,))
    return dy, h, ys, dhs


@traced_op("grouped_update_stage1", _update_stage1_fake)
def _update_stage1(W0_W2: Tensor, W1: Tensor, K: Tensor, V: Tensor, lr0: Optional[Tensor],
                   lr1: Optional[Tensor], lr2: Optional[Tensor], group_sizes: Tensor,
                   token_major: bool, save: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(DY0_DY2, Hidden) of the UPDATE, token-major ([B,N,2I], [B,N,I]) or the
    reference layout ([B,2I,N], [B,I,N]).  lr0 = lr1 = lr2 = None means lr = 1
    (the APPLY backward's pass with V = grad_out).  save: also return the
    bf16 (Y0 | Y2) [B,N,2I] and DH [B,N,I] the backward takes instead of
    recomputing them."""
    L.require_device(W0_W2, W1, K, V, lr0, lr1, lr2, group_sizes)
    _check_bf16(W0_W2, W1, K, V)
    B, E, I2, D = W0_W2.shape
    I = I2 // 2
    N = K.shape[1]
    assert K.shape == (B, N, D) and V.shape == (B, N, D)
    assert W1.shape == (B, E, D, I)
    lrs = []
    if lr0 is None:
        assert lr1 is None and lr2 is None
        lrs = [None, None, None]
        lr_code = L.F32
    else:
        for lr in (lr0, lr1, lr2):
            lr = lr.reshape(B, N) if lr.numel() == B * N else lr
            assert lr.shape == (B, N), f"lr must be [B, N], got {tuple(lr.shape)}"
            lrs.append(lr.contiguous())
        assert lrs[0].dtype == lrs[1].dtype == lrs[2].dtype
        lr_code = L.dtype_code(lrs[0].dtype)
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    dev = K.device
    if token_major:
        DY = torch.empty((B, N, I2), dtype=torch.bfloat16, device=dev)
        H = torch.empty((B, N, I), dtype=torch.bfloat16, device=dev)
    else:
        DY = torch.empty((B, I2, N), dtype=torch.bfloat16, device=dev)
        H = torch.empty((B, I, N), dtype=torch.bfloat16, device=dev)
    Ys = DHs = None
    if save:
        Ys = torch.empty((B, N, I2), dtype=torch.bfloat16, device=dev)
        DHs = torch.empty((B, N, I), dtype=torch.bfloat16, device=dev)
    else:
        Ys = torch.empty((0,), dtype=torch.bfloat16, device=dev)
        DHs = torch.empty((0,), dtype=torch.bfloat16, device=dev)
    ws_bytes = L.lib().uttt_update_stage1_workspace_bytes(B, I, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    L.call("uttt_grouped_update_stage1", L.ptr(W0_W2), L.ptr(W1), L.ptr(K), L.ptr(V),
           L.ptr(lrs[0]), L.ptr(lrs[1]), L.ptr(lrs[2]), lr_code, L.ptr(gs),
           B, E, I, D, N, L.ptr(DY), L.ptr(H), int(token_major), L.ptr(Ys) if save else None,
           L.ptr(DHs) if save else None, L.ptr(ws), ws_bytes, L.stream_of(K))
    return DY, H, Ys, DHs


def _wgrad_pair_fake(DY_tok, K, H_tok, V, group_sizes):
    B, N, I2 = DY_tok.shape
    E, D = group_sizes.shape[1], K.shape[2]
    return K.new_empty((B, E, I2, D)), K.new_empty((B, E, D, I2 // 2))


@traced_op("grouped_wgrad_pair", _wgrad_pair_fake)
def wgrad_pair(DY_tok: Tensor, K: Tensor, H_tok: Tensor, V: Tensor,
               group_sizes: Tensor) -> tuple[Tensor, Tensor]:
    """dW0_W2 [B,E,2I,D] = DY[seg]^T K[seg]; dW1 [B,E,D,I] = V[seg]^T H[seg]."""
    L.require_device(DY_tok, K, H_tok, V, group_sizes)
    _check_bf16(DY_tok, K, H_tok, V)
    B, N, I2 = DY_tok.shape
    I = I2 // 2
    D = K.shape[2]
    assert K.shape == (B, N, D) and V.shape == (B, N, D) and H_tok.shape == (B, N, I)
    gs = group_sizes_i32(group_sizes)
    E = gs.shape[1]
    dev = K.device
    dW02 = torch.empty((B, E, I2, D), dtype=torch.bfloat16, device=dev)
    dW1 = torch.empty((B, E, D, I), dtype=torch.bfloat16, device=dev)
    # split-K partials when few output tiles (one expert, small weights)
    nws = L.lib().uttt_grouped_wgrad_pair_workspace_bytes(B, E, I, D, N)
    ws = torch.empty(nws, dtype=torch.uint8, device=dev) if nws else None
    L.call("uttt_grouped_wgrad_pair", L.ptr(DY_tok), L.ptr(K), L.ptr(H_tok), L.ptr(V), L.ptr(gs),
           B, E, I, D, N, L.ptr(dW02), L.ptr(dW1), L.ptr(ws), nws, L.stream_of(K))
    return dW02, dW1


def _wgrad_fake(A_tok, B_tok, group_sizes, transposed):
    B, R, C, E = A_tok.shape[0], A_tok.shape[2], B_tok.shape[2], group_sizes.shape[1]
    return A_tok.new_empty((B, E, C, R) if transposed else (B, E, R, C))


@traced_op("grouped_wgrad", _wgrad_fake)
def wgrad(A_tok: Tensor, B_tok: Tensor, group_sizes: Tensor, transposed: bool) -> Tensor:
    """out[b,e] = A[seg]^T B[seg] as [B,E,R,C] (or [B,E,C,R] when transposed)."""
    L.require_device(A_tok, B_tok, group_sizes)
    _check_bf16(A_tok, B_tok)
    B, N, R = A_tok.shape
    C = B_tok.shape[2]
    assert B_tok.shape[:2] == (B, N)
    gs = group_sizes_i32(group_sizes)
    E = gs.shape[1]
    shape = (B, E, C, R) if transposed else (B, E, R, C)
    out = torch.empty(shape, dtype=torch.bfloat16, device=A_tok.device)
    L.call("uttt_grouped_wgrad", L.ptr(A_tok), L.ptr(B_tok), L.ptr(gs), B, E, R, C, N,
           L.ptr(out), int(transposed), L.stream_of(A_tok))
    return out


def _transpose_fake(X):
    return X.new_empty((X.shape[0], X.shape[2], X.shape[1]))


@traced_op("transpose_2byte", _transpose_fake)
def transpose_last2(X: Tensor) -> Tensor:
    """[B, R, C] -> [B, C, R] (2-byte elements) on the GPU."""
    L.require_device(X)
    assert X.element_size() == 2
    X = X.contiguous()
    B, R, C = X.shape
    out = torch.empty((B, C, R), dtype=X.dtype, device=X.device)
    L.call("uttt_transpose_2byte", L.ptr(X), B, R, C, L.ptr(out), L.stream_of(X))
    return out


def _gemm2(name, Wa, Xa, Wb, Xb, group_sizes, rows_first: bool):
    L.require_device(Wa, Xa, Wb, Xb, group_sizes)
    _check_bf16(Wa, Xa, Wb, Xb)
    assert Wa.shape == Wb.shape and Xa.shape == Xb.shape, "the two pairs must match in shape"
    B, E, R, C = Wa.shape
    M, K = (R, C) if rows_first else (C, R)
    Bx, N, Kx = Xa.shape
    assert Bx == B and Kx == K, "X must be [B, N, K] with matching B, K"
    gs = group_sizes_i32(group_sizes)
    assert gs.shape == (B, E)
    Y = torch.empty((B, N, M), dtype=torch.bfloat16, device=Xa.device)
    L.call(name, L.ptr(Wa), L.ptr(Xa), L.ptr(Wb), L.ptr(Xb), L.ptr(gs), B, E, M, K, N, L.ptr(Y),
           L.stream_of(Xa))
    return Y


def _gemm2_fake(Wa, Xa, Wb, Xb, group_sizes, rows_first):
    M = Wa.shape[2] if rows_first else Wa.shape[3]
    return Xa.new_empty((Xa.shape[0], Xa.shape[1], M))


def _gemm_nt2_fake(Wa, Xa, Wb, Xb, group_sizes):
    return _gemm2_fake(Wa, Xa, Wb, Xb, group_sizes, True)


def _gemm_tn2_fake(Wa, Xa, Wb, Xb, group_sizes):
    return _gemm2_fake(Wa, Xa, Wb, Xb, group_sizes, False)


@traced_op("grouped_gemm_nt2", _gemm_nt2_fake)
def gemm_nt2(Wa: Tensor, Xa: Tensor, Wb: Tensor, Xb: Tensor, group_sizes: Tensor) -> Tensor:
    """Y[b, n] = Wa[b, e(n)] Xa[b, n] + Wb[b, e(n)] Xb[b, n]: W [B,E,M,K] -> [B,N,M]."""
    return _gemm2("uttt_grouped_gemm_nt2", Wa, Xa, Wb, Xb, group_sizes, True)


@traced_op("grouped_gemm_tn2", _gemm_tn2_fake)
def gemm_tn2(Wa: Tensor, Xa: Tensor, Wb: Tensor, Xb: Tensor, group_sizes: Tensor) -> Tensor:
    """Y[b, n] = Wa[b, e(n)]^T Xa[b, n] + Wb[b, e(n)]^T Xb[b, n]: W [B,E,K,M] -> [B,N,M]."""
    return _gemm2("uttt_grouped_gemm_tn2", Wa, Xa, Wb, Xb, group_sizes, False)


def _swiglu_bwd_bwd_fake(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1):
    B, I, Lt = dh.shape
    xd, ld = x0_x2.dtype, lr0.dtype
    e = lambda *sh, dt: dh.new_empty(sh, dtype=dt)
    return (e(B, I, Lt, dt=xd), e(B, 2 * I, Lt, dt=xd), e(B, Lt, dt=ld), e(B, Lt, dt=ld),
            e(B, Lt, dt=ld), e(B, 2 * I, Lt, dt=xd), e(B, I, Lt, dt=xd))


@traced_op("swiglu_bwd_bwd", _swiglu_bwd_bwd_fake)
def swiglu_bwd_bwd(dh: Tensor, x0_x2: Tensor, lr0: Tensor, lr1: Tensor, lr2: Tensor,
                   grad_dx0_dx2: Tensor, grad_hidden_lr1: Tensor
                   ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Second-order SwiGLU pointwise pass on [B, I, L] / [B, 2I, L] tensors."""
    L.require_device(dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1)
    B, I, Lt = dh.shape
    assert x0_x2.shape == (B, 2 * I, Lt) and grad_dx0_dx2.shape == (B, 2 * I, Lt)
    assert grad_hidden_lr1.shape == (B, I, Lt)
    for t in (lr0, lr1, lr2):
        assert t.shape == (B, Lt), "lr tensors must be [B, L]"
    xd, ld = x0_x2.dtype, lr0.dtype
    assert dh.dtype == xd and grad_dx0_dx2.dtype == xd and grad_hidden_lr1.dtype == xd
    assert lr1.dtype == ld and lr2.dtype == ld
    ins = [t.contiguous() for t in (dh, x0_x2, lr0, lr1, lr2, grad_dx0_dx2, grad_hidden_lr1)]
    dev = dh.device
    g_dh = torch.empty((B, I, Lt), dtype=xd, device=dev)
    g_x = torch.empty((B, 2 * I, Lt), dtype=xd, device=dev)
    glr = [torch.empty((B, Lt), dtype=ld, device=dev) for _ in range(3)]
    dx = torch.empty((B, 2 * I, Lt), dtype=xd, device=dev)
    hl = torch.empty((B, I, Lt), dtype=xd, device=dev)
    ws_bytes = L.lib().uttt_swiglu_bwd_bwd_workspace_bytes(B, I, Lt)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    L.call("uttt_swiglu_bwd_bwd", L.ptr(ins[0]), L.ptr(ins[1]), L.dtype_code(xd), L.ptr(ins[2]),
           L.ptr(ins[3]), L.ptr(ins[4]), L.dtype_code(ld), L.ptr(ins[5]), L.ptr(ins[6]), B, I, Lt,
           L.ptr(g_dh), L.ptr(g_x), L.ptr(glr[0]), L.ptr(glr[1]), L.ptr(glr[2]), L.ptr(dx),
           L.ptr(hl), L.ptr(ws), ws_bytes, L.stream_of(dh))
    return g_dh, g_x, glr[0], glr[1], glr[2], dx, hl
