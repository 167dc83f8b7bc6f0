"""Oracle for the permute path (checker only; see oracle/__init__.py).

Integer and byte work (row map, permute, unpermute, permute_kv_and_lrs) is
the C restatement in permute_oracle.c, driven here through ctypes on numpy
buffers.  Backward passes are fp32 torch restatements of the reference's
backward kernels.

Reference: uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/
           triton_permute.py (P:line).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from . import build as _build

_lib = None
F32, BF16 = 0, 1


def _c():
    global _lib
    if _lib is None:
        path = _build.LIB
        if not os.path.exists(path):
            _build.build()
        _lib = ctypes.CDLL(path)
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _np(t: torch.Tensor) -> np.ndarray:
    """CPU contiguous numpy view; bf16 becomes its uint16 bit pattern."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _dtcode(dt):
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise ValueError(dt)


def _to_torch(a: np.ndarray, dtype) -> torch.Tensor:
    if dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(a)


def make_row_id_map(routing_map: torch.Tensor) -> torch.Tensor:
    """P:283-393 via the literal three-pass restatement."""
    B, E, T = routing_map.shape
    m = np.ascontiguousarray(_np(routing_map.to(torch.int32)))
    out = np.zeros((B, T, 2 * E + 1), dtype=np.int32)
    _c().oracle_make_row_id_map(_p(m), B, T, E, _p(out))
    return torch.from_numpy(out)


def meaningful_mask(row_id_map: torch.Tensor) -> torch.Tensor:
    """Entries the reference defines; all entries are defined (pass 3 leaves
    stale pass-2 values in [n, E) and zeros in [E+n, 2E))."""
    return torch.ones_like(row_id_map, dtype=torch.bool)


def permute(inp, row_id_map, probs, num_out, fill=0):
    """P:396-473.  Rows never written keep `fill` (the reference leaves them
    uninitialised; tests compare only the written rows)."""
    B, T, H = inp.shape
    E = (row_id_map.shape[-1] - 1) // 2
    x = np.ascontiguousarray(_np(inp))
    rm = np.ascontiguousarray(_np(row_id_map))
    out = np.full((B, num_out, H), fill, dtype=x.dtype)
    pp = None
    pr = None
    if probs is not None:
        pr = np.ascontiguousarray(_np(probs.float()))
        pp = np.zeros((B, num_out), dtype=np.float32)
    _c().oracle_permute(_p(x), ctypes.c_int(inp.element_size()), B, T, H, _p(rm), E, _p(pr),
                        _p(out), num_out, _p(pp))
    return _to_torch(out, inp.dtype), (None if pp is None else torch.from_numpy(pp))


def written_rows(row_id_map: torch.Tensor, num_out: int) -> torch.Tensor:
    """[B, num_out] bool: rows some token writes."""
    B, T, W = row_id_map.shape
    E = (W - 1) // 2
    n = row_id_map[..., 2 * E]
    res = torch.zeros(B, num_out, dtype=torch.bool)
    for j in range(E):
        sel = n > j
        rows = row_id_map[..., j]
        for b in range(B):
            r = rows[b][sel[b]].long()
            res[b, r] = True
    return res


def unpermute(inp, row_id_map, probs, num_tokens):
    """P:765-850 with fp32 fma accumulation in slot order."""
    B, num_out, H = inp.shape
    E = (row_id_map.shape[-1] - 1) // 2
    x = np.ascontiguousarray(_np(inp))
    rm = np.ascontiguousarray(_np(row_id_map))
    pr = None if probs is None else np.ascontiguousarray(_np(probs.float().contiguous()))
    out = np.zeros((B, num_tokens, H), dtype=x.dtype)
    _c().oracle_unpermute(_p(x), _dtcode(inp.dtype), B, num_out, H, _p(rm), num_tokens, E,
                          _p(pr), _p(out))
    return _to_torch(out, inp.dtype)


def permute_kv_lrs(k, v, lr0, lr1, lr2, row_id_map, probs, num_out):
    """P:1333-1493."""
    B, T, H = k.shape
    E = (row_id_map.shape[-1] - 1) // 2
    ka, va = np.ascontiguousarray(_np(k)), np.ascontiguousarray(_np(v))
    l0, l1, l2 = (np.ascontiguousarray(_np(x.reshape(B, T))) for x in (lr0, lr1, lr2))
    rm = np.ascontiguousarray(_np(row_id_map))
    pr = np.ascontiguousarray(_np(probs.float().contiguous()))
    ko = np.zeros((B, num_out, H), dtype=ka.dtype)
    vo = np.zeros((B, num_out, H), dtype=ka.dtype)
    lo = [np.zeros((B, num_out), dtype=l0.dtype) for _ in range(3)]
    _c().oracle_permute_kv_lrs(_p(ka), _dtcode(k.dtype), _p(va), _dtcode(v.dtype), _p(l0), _p(l1),
                               _p(l2), ctypes.c_int(lr0.element_size()), B, T, H, _p(rm), E,
                               _p(pr), _p(ko), _p(vo), _p(lo[0]), _p(lo[1]), _p(lo[2]), num_out)
    return (_to_torch(ko, k.dtype), _to_torch(vo, k.dtype),
            *(_to_torch(x, lr0.dtype) for x in lo))


def _slots(row_id_map):
    B, T, W = row_id_map.shape
    E = (W - 1) // 2
    return E, row_id_map[..., 2 * E]


def permute_bwd(grad_out, row_id_map, grad_pprobs, num_tokens):
    """P:579-680: grad_inp[t] = sum_j grad_out[row_j] (fp32, slot order);
    grad_probs[e_j, t] = grad_pprobs[row_j], else 0."""
    B, num_out, H = grad_out.shape
    E, n = _slots(row_id_map)
    g = grad_out.float()
    gi = torch.zeros(B, num_tokens, H)
    gp = torch.zeros(B, E, num_tokens) if grad_pprobs is not None else None
    for j in range(E):
        for b in range(B):
            sel = (n[b] > j).nonzero().flatten()
            rows = row_id_map[b, sel, j].long()
            gi[b, sel] += g[b, rows]
            if gp is not None:
                gp[b, row_id_map[b, sel, E + j].long(), sel] = grad_pprobs[b, rows].float()
    return gi.to(grad_out.dtype), gp


def unpermute_bwd(grad_out, row_id_map, fwd_inp, probs):
    """P:931-1058: act_grad[row_j] = cast(g[t] * p_j);
    grad_probs[e_j, t] = sum_h y[row_j, h] * g[t, h]; zero when not routed."""
    B, T, H = grad_out.shape
    num_out = fwd_inp.shape[1]
    E, n = _slots(row_id_map)
    g = grad_out.float()
    y = fwd_inp.float()
    pr = probs.float()
    ag = torch.zeros(B, num_out, H, dtype=grad_out.dtype)
    gp = torch.zeros(B, E, T)
    for j in range(E):
        for b in range(B):
            sel = (n[b] > j).nonzero().flatten()
            rows = row_id_map[b, sel, j].long()
            ex = row_id_map[b, sel, E + j].long()
            p = pr[b, ex, sel]
            ag[b, rows] = (g[b, sel] * p[:, None]).to(grad_out.dtype)
            gp[b, ex, sel] = (y[b, rows].double() * g[b, sel].double()).sum(-1).float()
    return ag, gp


def permute_kv_lrs_bwd(gk, gv, glr, row_id_map, v, probs, num_tokens):
    """P:1496-1727 (glr: list of three [B, num_out] grads)."""
    B, num_out, H = gk.shape
    E, n = _slots(row_id_map)
    pr = probs.float()
    gkf, gvf, vf = gk.float(), gv.float(), v.float()
    grad_k = torch.zeros(B, num_tokens, H)
    grad_v = torch.zeros(B, num_tokens, H)
    grad_lr = [torch.zeros(B, num_tokens) for _ in range(3)]
    gp = torch.zeros(B, E, num_tokens)
    for j in range(E):
        for b in range(B):
            sel = (n[b] > j).nonzero().flatten()
            rows = row_id_map[b, sel, j].long()
            ex = row_id_map[b, sel, E + j].long()
            p = pr[b, ex, sel]
            grad_k[b, sel] += gkf[b, rows]
            grad_v[b, sel] += gvf[b, rows] * p[:, None]
            for i in range(3):
                grad_lr[i][b, sel] += glr[i][b, rows].float()
            dot = (gvf[b, rows].double() * vf[b, sel].double()).sum(-1).float()
            gp[b, ex, sel] = torch.where(p == 0, torch.zeros_like(dot), dot)
    return grad_k.to(gk.dtype), grad_v.to(v.dtype), [g.to(glr[0].dtype) for g in grad_lr], gp
