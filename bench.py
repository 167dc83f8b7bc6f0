#!/usr/bin/env python3
"""Benchmark of uTTT's fast-weight hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line (rank 0).  Workloads (seeded synthetic inputs, resident
in HBM before the timed region starts):

  moe760m   (default) configs[4]: uTTT-MoE 760M training slice, E=32 experts,
            top-2, d=1536, expert hidden 3072, Zipf(1.1) routing prior, 24
            layers sharing the pool, seq 32768 in chunks of 2048.  One step =
            one shifted block-causal sweep: APPLY (row map, permute, grouped
            SwiGLU apply, unpermute) on 16 chunks x 24 layers, UPDATE forward
            and backward on 15 x 24, the router in front of every APPLY and
            UPDATE and the norm-preserving WRITE after every UPDATE; value =
            tokens/s of the sweep.
  moe124m   configs[3]: uTTT-MoE 124M, E=16, d=768, hidden 1536, 12 layers,
            APPLY + UPDATE forward + WRITE.
  dense124m configs[1]: uTTT-Dense 124M, one shared SwiGLU fast weight per
            head (H=4, d=192, hidden 384), 12 layers, aggregate write.
  dense_c0  configs[0]'s single-layer shape (H=4, d=96, hidden 192, chunks of
            512) on the GPU.
  decode760m generation-time read at the 760M shape: 8 sequences with their
            own pools, one token each through 24 layers (router + routed
            SwiGLU read); value = tokens/s.
  muon760m  the Muon write of one chunk on the 760M pool (momentum,
            Newton-Schulz5 of the 96 expert matrices, scaled add,
            norm-preserving write); value = NS5 algorithmic TFLOP/s.
  permute   configs[2]: token permute + gate-weighted unpermute by expert,
            T=65536, E=16, top-2, payload bf16 [T, 768]; one step = row map +
            permute + unpermute of one batch; value = algorithmic GB/s.

Timing: W untimed steps, then K steps bracketed by torch.cuda.synchronize().
The MoE sweeps run through the product API (uttt_amd.moe, the compat ops
under it, autograd for the UPDATE backward, uttt_amd.fast_weight_write).
`kernels_by_symbol` groups one more sweep's GPU time by kernel symbol (from
torch.profiler's device activity); `roofline` reports the symbol with the
most time per sweep against MI355X's published peak, with its launch time
measured by HIP events around back-to-back launches on the launch stream;
`cpu_baseline` times the CPU restatement under oracle/ on all of this host's
cores (rank 0, N=1; 1 warm-up, median of 3) on a bounded sample of the same
workload.  The default line also carries `other_targets`: configs[2]'s
permute / unpermute GB/s, configs[3]'s sweep, and the uTTT-Dense sweeps of
configs[1] and configs[0]'s shape.

Only one GPU is used: --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s


def _events(n):
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


# --------------------------------------------------------------- permute ----
def _routing(T, E, k, seed, device, zipf=None):
    """Router draw of the permute microbench: logits ~ N(0,1) [1,E,T], a
    per-expert selection bias ~ N(0, 0.5) (or a Zipf prior), top-k over the
    biased scores, gates = softmax over E restricted to the top-k and
    renormalised ("topk_renorm").  Input generation only (plain torch)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(1, E, T, generator=g)
    if zipf is not None:
        bias = (-zipf * torch.log(torch.arange(E, dtype=torch.float32) + 1.0)).view(1, E, 1)
    else:
        bias = (torch.randn(E, generator=g) * 0.5).view(1, E, 1)
    logits, bias = logits.to(device), bias.to(device)
    idx = torch.topk(logits + bias, k, dim=1).indices
    mask = torch.zeros_like(logits, dtype=torch.bool).scatter_(1, idx, True)
    sm = torch.softmax(logits, dim=1) * mask
    gates = sm / sm.sum(dim=1, keepdim=True).clamp_min(1e-9)
    return mask, gates, g


def _profile_traffic(summary, kernel):
    """HBM bytes per launch of `kernel` as measured by the rocprofv3 PMC passes
    (FETCH_SIZE and WRITE_SIZE, scaled by the copy calibration) recorded in
    profiles/<summary> ("traffic_bytes <kernel> <bytes>"); None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", summary)
    try:
        with open(path) as f:
            for line in f:
                if not line.startswith("traffic_bytes "):
                    continue
                name, value = line[len("traffic_bytes "):].rstrip().rsplit(None, 1)
                if name == kernel:  # kernel names may hold spaces
                    return int(value)
    except OSError:
        pass
    return None


def bench_permute(args):
    import torch

    from uttt_amd import _lib as L

    dev = torch.device("cuda", 0)
    B, T, E, k, D = 1, 65536, 16, 2, 768
    nsets = 3  # rotate buffer sets so consecutive steps do not hit in MALL
    sets = []
    for s in range(nsets):
        mask, gates, g = _routing(T, E, k, seed=s, device=dev)
        x = torch.randn(B, T, D, generator=g).to(torch.bfloat16).to(dev)
        sets.append(
            dict(
                mask=mask,
                gates=gates.contiguous(),
                x=x,
                rmap=torch.empty(B, T, 2 * E + 1, dtype=torch.int32, device=dev),
                gs=torch.empty(B, E, dtype=torch.int32, device=dev),
                xp=torch.empty(B, k * T, D, dtype=torch.bfloat16, device=dev),
                pp=torch.empty(B, k * T, dtype=torch.float32, device=dev),
                y=torch.empty(B, T, D, dtype=torch.bfloat16, device=dev),
            )
        )
    ws_bytes = L.lib().uttt_row_id_map_workspace_bytes(B, T, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    BF16 = L.BF16

    def rowmap(s):
        L.call("uttt_make_row_id_map", L.ptr(s["mask"]), 1, s["mask"].stride(0),
               s["mask"].stride(1), s["mask"].stride(2), B, T, E, L.ptr(s["rmap"]),
               L.ptr(s["gs"]), L.ptr(ws), ws_bytes, stream)

    def permute(s):
        p = s["gates"]
        L.call("uttt_permute_fwd", L.ptr(s["x"]), BF16, B, T, D, L.ptr(s["rmap"]), E,
               L.ptr(p), p.stride(0), p.stride(1), p.stride(2), L.ptr(s["xp"]), k * T,
               L.ptr(s["pp"]), stream)

    def unpermute(s):
        p = s["gates"]
        L.call("uttt_unpermute_fwd", L.ptr(s["xp"]), BF16, B, k * T, D, L.ptr(s["rmap"]), T, E,
               L.ptr(p), p.stride(0), p.stride(1), p.stride(2), L.ptr(s["y"]), stream)

    def step(s):
        rowmap(s)
        permute(s)
        unpermute(s)

    def timed(fn, reps):
        """Mean duration of `reps` back-to-back launches over the rotating
        buffer sets, between two events on the launch stream."""
        e0, e1 = _events(2)
        e0.record()
        for i in range(reps):
            fn(sets[i % nsets])
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps

    for i in range(args.warmup):
        step(sets[i % nsets])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_step = timed(step, args.steps)
    wall = time.perf_counter() - t0
    reps = max(3 * args.steps, 30)
    t_map = timed(rowmap, reps)
    t_p = timed(permute, reps)

    def rowmap_permute(s):   # what permute_with_expert_mask runs (L/triton_permute.py:1184-1187)
        rowmap(s)
        permute(s)

    t_mp = timed(rowmap_permute, reps)
    t_u = timed(unpermute, reps)
    # practical streaming ceiling on the same buffers: a plain device copy
    t_copy = timed(lambda s: s["y"].copy_(s["x"]), reps)

    # algorithmic bytes (each tensor once): permute reads x and the k row ids
    # per token and writes k copies; unpermute reads the k rows, their gates
    # and row ids, and writes one row per token.
    row = D * 2
    perm_bytes = T * row + k * T * 4 + k * T * row
    unp_bytes = k * T * row + k * T * (4 + 4) + T * row
    map_bytes = E * T * 1 + T * (2 * E + 1) * 4
    step_bytes = perm_bytes + unp_bytes
    value = (step_bytes + map_bytes) / t_step / 1e9

    # sanity: the HIP path ran and produced the unpermute∘permute invariant
    s = sets[(args.steps - 1) % nsets]
    m = s["mask"].float()
    ref = (s["x"].float() * (s["gates"] * m).sum(1).unsqueeze(-1))
    err = (s["y"].float() - ref).abs().max().item()
    assert err < 2e-2 * ref.abs().max().item() + 1e-3, f"permute/unpermute invariant broken: {err}"

    res = dict(
        metric="permute+unpermute GB/s (algorithmic bytes)",
        value=round(value, 2),
        unit="GB/s",
        ms_per_step=round(t_step * 1e3, 4),
        wall_ms_per_step=round(wall / args.steps * 1e3, 4),
        dtype="bf16",
        config={"workload": "uttt-moe permute/unpermute microbench (configs[2])", "T": T, "E": E,
                "topk": k, "hidden": D, "payload": "bf16", "buffer_sets": nsets},
        roofline=dict(
            bound="hbm", kernel="permute_chunk_kernel",
            achieved=round(perm_bytes / t_p / 1e9, 2), peak=HBM_PEAK_GBS, unit="GB/s",
            frac=round(perm_bytes / t_p / 1e9 / HBM_PEAK_GBS, 4),
            traffic=_profile_traffic("permute_unpermute_c2.txt", "permute_chunk_kernel"),
            algorithmic_bytes=perm_bytes, avg_launch_us=round(t_p * 1e6, 3),
        ),
        permute_end_to_end=dict(
            us=round(t_mp * 1e6, 3), GBs=round((perm_bytes + map_bytes) / t_mp / 1e9, 1),
            hbm_frac=round((perm_bytes + map_bytes) / t_mp / 1e9 / HBM_PEAK_GBS, 4),
            what="permute_with_expert_mask as one call: the row map from the mask, then the "
                 "permute (algorithmic bytes of both)"),
        kernels={
            "row_id_map": dict(us=round(t_map * 1e6, 3), GBs=round(map_bytes / t_map / 1e9, 1)),
            "permute_chunk_kernel": dict(us=round(t_p * 1e6, 3), GBs=round(perm_bytes / t_p / 1e9, 1),
                                       hbm_frac=round(perm_bytes / t_p / 1e9 / HBM_PEAK_GBS, 4)),
            "device_copy(x -> y)": dict(us=round(t_copy * 1e6, 3),
                                        GBs=round(2 * T * row / t_copy / 1e9, 1)),
            "unpermute_chunk_kernel": dict(us=round(t_u * 1e6, 3),
                                         GBs=round(unp_bytes / t_u / 1e9, 1),
                                         hbm_frac=round(unp_bytes / t_u / 1e9 / HBM_PEAK_GBS, 4)),
        },
    )
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_permute(sets[0], B, T, E, k, D, step_bytes + map_bytes)
    return res


def cpu_baseline_permute(s, B, T, E, k, D, step_bytes):
    """The C restatement of the permute path (oracle/permute_oracle.c, single
    thread) on the same inputs: row map + permute + unpermute, repeated for
    about 10 s of CPU work."""
    import numpy as np
    import torch

    from oracle import permute as OP

    mask = s["mask"].cpu().to(torch.int32).contiguous()
    gates = s["gates"].cpu().contiguous()
    x = s["x"].cpu()
    lib = OP._c()
    m = mask.numpy()
    xa = x.view(torch.int16).numpy()
    ga = gates.numpy()
    rm = np.zeros((B, T, 2 * E + 1), dtype=np.int32)
    xp = np.zeros((B, k * T, D), dtype=np.int16)
    pp = np.zeros((B, k * T), dtype=np.float32)
    y = np.zeros((B, T, D), dtype=np.int16)
    P = OP._p
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        lib.oracle_make_row_id_map(P(m), B, T, E, P(rm))
        lib.oracle_permute(P(xa), ctypes.c_int(2), B, T, D, P(rm), E, P(ga), P(xp), k * T, P(pp))
        lib.oracle_unpermute(P(xp), 1, B, k * T, D, P(rm), T, E, P(ga), P(y))
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 10.0 and len(times) >= 3:
            break
    t = statistics.median(times)
    return dict(value=round(step_bytes / t / 1e9, 3), unit="GB/s", cores=1, kind="port",
                sample=f"full configs[2] step (row map + permute + unpermute, T={T}), "
                       f"{len(times)} repeats, median {t * 1e3:.1f} ms",
                cpu=_cpu_model())


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_calibration():
    """One plain device copy of a known size (256 MiB read + 256 MiB write),
    used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings."""
    import torch

    n = 256 * 1024 * 1024
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(f"copy_calibration: {n} bytes read, {n} bytes written", file=sys.stderr)


# ------------------------------------------------------------ MoE sweep ----
MOE_CONFIGS = {
    # uTTT-MoE 124M, apply + update forward, 12 layers share the pool
    "moe124m": dict(E=16, D=768, I=1536, L=12, zipf=None, train=False,
                    label="uTTT-MoE 124M grouped apply+update (configs[3])"),
    # uTTT-MoE 760M training slice: apply fwd + update fwd + update bwd
    "moe760m": dict(E=32, D=1536, I=3072, L=24, zipf=1.1, train=True,
                    label="uTTT-MoE 760M apply+update fwd+bwd training slice (configs[4])"),
    # configs[4] with the shipped configs' write: momentum and Muon (use_momentum,
    # use_moun of uttt_llm/configs/main/760M/uttt_moe.json)
    "moe760m_shipped": dict(E=32, D=1536, I=3072, L=24, zipf=1.1, train=True, shipped=True,
                            label="uTTT-MoE 760M training slice (configs[4]) with the shipped "
                                  "write: momentum + Muon (Newton-Schulz per expert matrix)"),
}
SEQ, CHUNK, TOPK = 32768, 2048, 2


def norm_symbol(name):
    """A kernel's symbol without namespaces, argument list or return type:
    'tn_kernel<0, EpiSwiGLU, true>'."""
    import re

    s = name.replace("(anonymous namespace)::", "").replace("anon::", "").replace("uttt::", "")
    s = re.sub(r"^void\s+", "", s)
    depth, cut = 0, len(s)
    for i, ch in enumerate(s):          # drop a trailing "(...)" parameter list
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    s = s[:cut].strip()
    # wg_kernel<SPLIT, layout, LAYERED>: the plain weight gradients keep the
    # name 'wg_kernel<SPLIT>' whichever layout they run, the per-layer-operand
    # form becomes 'wg_kernel<SPLIT, layered>'
    m = re.match(r"^wg_kernel<(\w+), [12], (true|false)>$", s)
    if m:
        return f"wg_kernel<{m.group(1)}{', layered' if m.group(2) == 'true' else ''}>"
    # the GEMM kernels' last template argument is the wave layout (4 or 8
    # waves): one symbol per product family whichever layout it runs
    return re.sub(r"^((?:tn|wg)_kernel<.*), [12]>$", r"\1>", s)


class MoeSweep:
    """One shifted block-causal sweep over the sequence through the product
    API (uttt_amd.moe and uttt_amd.fast_weight_write), as a caller of the
    reference's model would drive it:
      - every (chunk, layer): the routed APPLY,
        moe.apply_moe_fast_weights_grouped (router -> row map -> permute ->
        grouped SwiGLU apply -> gate-weighted unpermute);
      - every chunk but the last: the UPDATE of the chunk's writers -- batched
        (the aggregate write: all L writers' tokens routed in one router launch,
        moe.route_writers, and summed by one grouped UPDATE,
        moe.aggregate_moe_update_grads) or per layer (one UPDATE per writer);
        for the training slice, its backward through autograd seeded with fixed
        upstream weight gradients (UPDATE backward and the permute's backward);
        then the norm-preserving WRITE of the pool
        (fast_weight_write.apply_moe_update_packed)."""

    NSETS = 4   # distinct per-layer input sets, cycled over (chunk, layer)

    def __init__(self, cfg, dev):
        import torch

        from uttt_amd import moe

        self.cfg, self.dev = cfg, dev
        E, D, I = cfg["E"], cfg["D"], cfg["I"]
        T, k = CHUNK, TOPK
        self.E, self.D, self.I, self.T, self.k, self.N = E, D, I, T, k, k * T
        g = torch.Generator(device=dev).manual_seed(0)
        bf = torch.bfloat16

        def randn(*shape, scale=1.0):
            return (torch.randn(*shape, generator=g, device=dev) * scale).to(bf)

        # the shared expert pool (W0_W2 = w0 rows then w2 rows, W1 = down proj)
        self.W02 = randn(1, E, 2 * I, D, scale=D ** -0.5)
        self.W1 = randn(1, E, D, I, scale=D ** -0.5)
        # fp32 masters of the pool for the WRITE step
        self.M02, self.M1 = self.W02.float(), self.W1.float()
        self.sets = []
        for _ in range(self.NSETS):
            st = {}
            for name in ("x", "k", "v"):
                t = torch.randn(1, T, D, generator=g, device=dev)
                st[name] = (t / (t.norm(dim=-1, keepdim=True) + 1e-5)).to(bf)
            st["lr"] = torch.sigmoid(torch.randn(1, T, 3, generator=g, device=dev)) * 0.1
            self.sets.append(st)
        # one router shared by all layers ("share_all"): logits = R x with x
        # L2-normalised and R ~ N(0, 1), so logits ~ N(0, 1); the expert prior
        # (Zipf for configs[4], N(0, 0.5) otherwise) is the selection-only
        # routing bias; gates are top-k renormalised
        self.R = torch.randn(E, D, generator=g, device=dev)
        if cfg["zipf"] is not None:
            self.rbias = -cfg["zipf"] * torch.log(torch.arange(E, device=dev, dtype=torch.float32) + 1)
        else:
            self.rbias = torch.randn(E, generator=g, device=dev) * 0.5
        self.rcfg = moe.RouterConfig(topk=k, combine_mode="topk_renorm")
        if cfg["train"]:
            self.GW02 = randn(1, E, 2 * I, D, scale=0.02)
            self.GW1 = randn(1, E, D, I, scale=0.02)
        self.shipped = bool(cfg.get("shipped"))
        if self.shipped:
            # momentum buffers of the pool and per-write coefficients
            # (momentum_proj's sigmoid, averaged over the chunk's tokens)
            self.MOM02, self.MOM1 = torch.zeros_like(self.M02), torch.zeros_like(self.M1)
            self.mcoeffs = torch.sigmoid(torch.randn(SEQ // CHUNK, 1, generator=g, device=dev))
            self.n_writes = 0
        self.marks = None   # [(name, event)] when the stages are bracketed

    def _mark(self, name):
        if self.marks is not None:
            import torch

            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self.marks.append((name, ev))

    def apply(self, st):
        import torch

        from uttt_amd import moe

        self._mark("apply")
        with torch.no_grad():
            out, _ = moe.apply_moe_fast_weights_grouped(
                st["x"], None, self.W1, None, self.R, self.rcfg, 1, routing_bias=self.rbias,
                precomputed_w0_w2=self.W02)
        return out

    def _grads(self, writers_k, writers_v, writers_lr, layers):
        """UPDATE (+ backward) of `layers` writers given as lists; returns the
        packed bf16 weight gradients."""
        import torch

        from uttt_amd import moe

        train = self.cfg["train"]
        self._mark("update_fwd")
        cat = (lambda ts: ts[0]) if layers == 1 else (lambda ts: torch.cat(ts, dim=1))
        K, V, LR = cat(writers_k), cat(writers_v), cat(writers_lr)
        if train:
            K, V, LR = (t.detach().requires_grad_() for t in (K, V, LR))
        with torch.no_grad():
            m, gs, p, _ = moe.route_writers(K.detach(), layers, self.R, self.rcfg,
                                            routing_bias=self.rbias)
        with torch.enable_grad() if train else torch.no_grad():
            dW02, dW1 = moe.aggregate_moe_update_grads(
                [moe.WriterInputs(K, V, LR, m, p)], None, self.W1, None, self.k,
                precomputed_w0_w2=self.W02, packed=True)
            if train:
                self._mark("update_bwd")
                torch.autograd.backward([dW02, dW1], [self.GW02, self.GW1])
        return dW02.detach(), dW1.detach()

    def write(self, dW02, dW1):
        from uttt_amd import fast_weight_write as FWW

        self._mark("write")
        if not self.shipped:
            FWW.apply_moe_update_packed(dW02, dW1, self.M02, self.M1, lr_scale=1.0,
                                        out=((self.W02, self.W1), (self.M02, self.M1)))
            return
        c = self.mcoeffs[self.n_writes % self.mcoeffs.shape[0]]
        self.n_writes += 1
        _, _, (self.MOM02, self.MOM1) = FWW.apply_moe_update_packed(
            dW02, dW1, self.M02, self.M1, momentum_buf=(self.MOM02, self.MOM1), m_coeff=c,
            lr_scale=1.0, use_momentum=True, use_moun=True,
            out=((self.W02, self.W1), (self.M02, self.M1)))

    def update_batched(self, layers, first_set):
        sets = [self.sets[(first_set + l) % self.NSETS] for l in range(layers)]
        dW02, dW1 = self._grads([s["k"] for s in sets], [s["v"] for s in sets],
                                [s["lr"] for s in sets], layers)
        self.write(dW02, dW1)

    def update_one(self, st):
        dW02, dW1 = self._grads([st["k"]], [st["v"]], [st["lr"]], 1)
        self.write(dW02, dW1)

    def sweep(self, layers, chunks, batched):
        i = 0
        for c in range(chunks):
            for _ in range(layers):
                self.apply(self.sets[i % self.NSETS])
                i += 1
            if c < chunks - 1:   # the last chunk is read but never written
                if batched:   # aggregate: all writers' gradients, one write
                    self.update_batched(layers, i)
                    i += layers
                else:         # chained: each writer updates and writes in turn
                    for _ in range(layers):
                        self.update_one(self.sets[i % self.NSETS])
                        i += 1
        self._mark(None)

    def capture_reads(self, layers):
        """One HIP graph (torch.cuda.CUDAGraph) of a chunk's `layers` routed
        reads through the product API.  Every chunk reads the same input sets
        (layers is a multiple of NSETS) and the pool in place, so the graph
        replays the reads of any chunk; the writes between replays update the
        buffers it reads."""
        import torch

        assert layers % self.NSETS == 0 and self.marks is None
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):   # allocations of the first calls outside the capture
            for l in range(layers):
                self.apply(self.sets[l % self.NSETS])
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for l in range(layers):
                self.apply(self.sets[l % self.NSETS])
        torch.cuda.synchronize()
        self.read_graph = graph

    def sweep_graphed(self, layers, chunks, batched):
        """sweep() with each chunk's routed reads replayed from capture_reads'
        graph (the updates and writes run eagerly between the replays)."""
        i = 0
        for c in range(chunks):
            self.read_graph.replay()
            i += layers
            if c < chunks - 1:
                if batched:
                    self.update_batched(layers, i)
                    i += layers
                else:
                    for _ in range(layers):
                        self.update_one(self.sets[i % self.NSETS])
                        i += 1

    # ---------------------------------------------------------- accounting --
    def apply_symbols(self):
        """Kernel symbols of the APPLY's gate/up and down projection, as the
        library picks them by the sizes: gate/up on the skinny tiles when the
        experts average at most 256 routed rows; the down projection on them
        when also the general 256x256 tiles would not fill the 256 CUs once
        (upper-bound tile count), else on the general tiles (their MFMA-skipping
        variant below 256 rows per expert)."""
        N, E, D = self.N, self.E, self.D
        skinny = N <= 256 * E
        gate = "apply_kernel<ApSwiGLU, true>" if skinny else "tn_kernel<0, EpiSwiGLU, false>"
        tn_tiles = -(-D // 256) * (-(-N // 256) + E)
        if skinny and tn_tiles < 256:
            down = "apply_kernel<ApStore, false>"
        else:
            skip = "true" if N < 256 * E else "false"
            down = f"tn_kernel<0, EpiStore<unsigned short, true>, {skip}>"
        return gate, down

    def launch_table(self, layers, chunks, batched):
        """Every kernel launch of one sweep that carries GEMM work, grouped by
        kernel symbol: {symbol: [algorithmic FLOP per sweep, algorithmic HBM
        bytes per sweep, launches per sweep]} (NID = rows * I * D of the call;
        bytes count each tensor once: the pool, token rows in and out)."""
        E, D, I = self.E, self.D, self.I
        Na = self.N
        Nu = self.N * (layers if batched else 1)
        n_apply = layers * chunks
        n_upd = (chunks - 1) * (1 if batched else layers)
        skip_u = "true" if Nu < 256 * E else "false"
        w_bytes = 2 * 3 * E * I * D
        tab = {}

        def add(sym, nid_mult, rows, n, bytes_):
            t = tab.setdefault(sym, [0, 0, 0])
            t[0] += nid_mult * rows * I * D * n
            t[1] += bytes_ * n
            t[2] += n

        gate_sym, down_sym = self.apply_symbols()
        add(gate_sym, 4, Na, n_apply, 2 * (E * 2 * I * D + Na * D + Na * I))
        add(down_sym, 2, Na, n_apply, 2 * (E * D * I + Na * I + Na * D))
        add("tn_kernel<1, EpiStore<float, true>, false>", 2, Nu, n_upd,
            2 * E * D * I + 2 * Nu * D + 4 * Nu * I)
        add("tn_kernel<0, EpiS1<BF16T>, false>", 4, Nu, n_upd,
            2 * E * 2 * I * D + 2 * Nu * D + 4 * Nu * I + 2 * 3 * Nu * I)
        add("wg_kernel<false>", 6, Nu, n_upd, w_bytes + 2 * Nu * (3 * I + 2 * D))
        if self.cfg["train"]:
            # the backward from the forward's saved bf16 Y0 | Y2 and DH
            add("tn_kernel<1, EpiStore<unsigned short, true>, false>", 2, Nu, n_upd,
                2 * E * D * I + 2 * Nu * D + 2 * Nu * I)                  # GD
            add("tn_kernel<0, EpiBwdSaved<BF16T>, false>", 4, Nu, n_upd,
                2 * E * 2 * I * D + 2 * Nu * D + 2 * Nu * 16 * I)         # GY + 2nd order
            add("tn_kernel<1, EpiStore<unsigned short, true>, false>", 8, Nu, n_upd,
                2 * 2 * E * 2 * I * D + 2 * Nu * 4 * I + 2 * Nu * D)      # grad_K
            add(f"tn_kernel<0, EpiStore<unsigned short, true>, {skip_u}>", 4, Nu, n_upd,
                2 * 2 * E * D * I + 2 * Nu * 2 * I + 2 * Nu * D)          # grad_V
            add("wg_kernel<false>", 6, Nu, n_upd, w_bytes + 2 * Nu * (3 * I + 2 * D))
        return tab

    def isolated(self, symbol, batched, reps=5):
        """Mean duration of `reps` back-to-back launches of one kernel symbol at
        the shape the sweep runs it, between two HIP events on the launch
        stream; None when this symbol has no single-launch recipe."""
        import torch

        from uttt_amd import _lib as L
        from uttt_amd import moe
        from uttt_amd.lact_moe_triton import _grouped
        from uttt_amd.lact_moe_triton.triton_permute import (permute_kv_and_lrs,
                                                             permute_with_expert_mask)

        E, D, I, s = self.E, self.D, self.I, torch.cuda.current_stream().cuda_stream
        gate_sym, down_sym = self.apply_symbols()
        upd = self.launch_table(self.cfg["L"], 2, batched)
        with torch.no_grad():
            if symbol == gate_sym or (symbol == down_sym and upd[down_sym][2] == 2 * self.cfg["L"]):
                st = self.sets[0]
                m, gs, p, _ = moe.route(st["x"], self.R, self.rcfg, routing_bias=self.rbias)
                xp, _, _ = permute_with_expert_mask(st["x"], m, p, self.k)
                N = xp.shape[1]
                hid = torch.empty(1, N, I, dtype=torch.bfloat16, device=self.dev)
                yp = torch.empty(1, N, D, dtype=torch.bfloat16, device=self.dev)
                if symbol == gate_sym:
                    fn = lambda: L.call("uttt_grouped_gate_up", L.ptr(self.W02), L.ptr(xp),
                                        L.ptr(gs), 1, E, I, D, N, L.ptr(hid), 1, s)
                else:
                    L.call("uttt_grouped_gate_up", L.ptr(self.W02), L.ptr(xp), L.ptr(gs), 1, E,
                           I, D, N, L.ptr(hid), 1, s)
                    fn = lambda: L.call("uttt_grouped_gemm_nt", L.ptr(self.W1), L.ptr(hid),
                                        L.ptr(gs), 1, E, D, I, N, L.ptr(yp), s)
            elif symbol == "wg_kernel<false>":
                layers = self.cfg["L"] if batched else 1
                sets = [self.sets[l % self.NSETS] for l in range(layers)]
                K = torch.cat([x["k"] for x in sets], 1)
                V = torch.cat([x["v"] for x in sets], 1)
                LR = torch.cat([x["lr"] for x in sets], 1)
                m, gs, p, _ = moe.route_writers(K, layers, self.R, self.rcfg,
                                                routing_bias=self.rbias)
                lrs = [LR[:, :, j].contiguous().to(torch.bfloat16) for j in range(3)]
                kp, vp, l0, l1, l2 = permute_kv_and_lrs(K, V, *lrs, m, p, self.k)
                dy, hl = _grouped.update_stage1(self.W02, self.W1, kp, vp, l0, l1, l2, gs,
                                                token_major=True)
                N = kp.shape[1]
                dW02 = torch.empty_like(self.W02)
                dW1 = torch.empty_like(self.W1)
                nws = L.lib().uttt_grouped_wgrad_pair_workspace_bytes(1, E, I, D, N)
                ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=self.dev)
                fn = lambda: L.call("uttt_grouped_wgrad_pair", L.ptr(dy), L.ptr(kp), L.ptr(hl),
                                    L.ptr(vp), L.ptr(gs), 1, E, I, D, N, L.ptr(dW02),
                                    L.ptr(dW1), L.ptr(ws), nws, s)
            else:
                return None
            fn()
            e0, e1 = _events(2)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps


def kernel_times_profiled(run):
    """{symbol: [total us, launches]} of the GPU kernels `run()` launches,
    from torch.profiler's device activity (the ROCm tracer's per-dispatch
    start and end); None when the profiler records no device activity."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        run()
        torch.cuda.synchronize()
    out = {}
    for ev in prof.events():
        if getattr(ev, "device_type", None) != torch.autograd.DeviceType.CUDA:
            continue
        us = ev.time_range.end - ev.time_range.start
        if us <= 0:
            continue
        d = out.setdefault(norm_symbol(ev.name), [0.0, 0])
        d[0] += us
        d[1] += 1
    return out or None


def kernel_times_from_profile(summary):
    """Fallback: {symbol: [total us, launches]} per sweep from the committed
    rocprofv3 summary profiles/<summary> ("<symbol> calls= n avg_us= t")."""
    import re

    path = os.path.join(ROOT, "profiles", summary)
    out = {}
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*(\S.*?)\s+calls=\s*(\d+)\s+avg_us=\s*([\d.]+)", line)
                if m:
                    out[norm_symbol(m.group(1))] = [float(m.group(3)) * int(m.group(2)),
                                                    int(m.group(2))]
    except OSError:
        return None
    return out or None


def _profile_value(summary, key, symbol):
    """A "<key> <symbol> <value>" line of profiles/<summary>, or None."""
    path = os.path.join(ROOT, "profiles", summary)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + " ") and line[len(key) + 1:].rsplit(" ", 1)[0] == symbol:
                    return float(line.rsplit(" ", 1)[1])
    except OSError:
        pass
    return None


def _stage_times(marks):
    """{stage: total seconds} from consecutive (name, event) marks."""
    out = {}
    for (name, ev), (_, ev2) in zip(marks, marks[1:]):
        if name is not None:
            out[name] = out.get(name, 0.0) + ev.elapsed_time(ev2) * 1e-3
    return out


def bench_moe(args, key, extras=True):
    import torch

    cfg = MOE_CONFIGS[key]
    dev = torch.device("cuda", 0)
    sw = MoeSweep(cfg, dev)
    layers, chunks = cfg["L"], SEQ // CHUNK
    batched = args.update_schedule == "batched"
    for _ in range(max(args.warmup, 1)):
        sw.sweep(layers, 2, batched)
    torch.cuda.synchronize()
    walls = []
    with LiveLaunchTimer(sw.apply_symbols()) as live:
        for _ in range(args.steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            sw.sweep(layers, chunks, batched)
            torch.cuda.synchronize()
            walls.append(time.perf_counter() - t0)
    wall = statistics.mean(walls)
    tokens = SEQ  # B = 1
    nid = sw.N * sw.I * sw.D
    # the reference's work per update (BASELINE: 12 NID, +30 NID backward) and
    # what this build executes (its backward reuses the forward's Y0, Y2, DH)
    sweep_flops = layers * (chunks * 6 + (chunks - 1) * (42 if cfg["train"] else 12)) * nid
    exec_flops = layers * (chunks * 6 + (chunks - 1) * (36 if cfg["train"] else 12)) * nid
    res = dict(
        metric="fast-weight apply+update tokens/s",
        value=round(tokens / wall, 1),
        unit="tokens/s",
        ms_per_step=round(wall * 1e3, 3),
        dtype="bf16",
        config={"workload": cfg["label"], "seq_len": SEQ, "chunk": CHUNK, "layers": layers,
                "experts": cfg["E"], "topk": TOPK, "d": cfg["D"], "expert_hidden": cfg["I"],
                "step": "one sweep: apply on 16 chunks x L layers, update on 15 chunks x L writers"
                        + (" (+ update backward)" if cfg["train"] else "") + " + write",
                "path": "product API: uttt_amd.moe (routed read, batched-writer routing and "
                        "aggregate update, autograd backward) + fast_weight_write",
                "update_schedule": ("batched: the L writers of a chunk in one grouped UPDATE "
                                    "call (aggregate write = sum of writer gradients)"
                                    if batched else "per-layer: one UPDATE call per writer"),
                "write": "norm-preserving write of the pool after every update "
                         "(fp32 masters, bf16 fast weights)",
                "routing": ("fused router per apply (x) and per update (k): fp32 logits of one "
                            "shared router, " + ("Zipf(1.1)" if cfg["zipf"] else "N(0,0.5)")
                            + " expert prior as selection bias, topk_renorm gates")},
        sweep=dict(algorithmic_flops=sweep_flops,
                   TFLOPs=round(sweep_flops / wall / 1e12, 1),
                   mfma_frac=round(sweep_flops / wall / 1e12 / BF16_PEAK_TFLOPS, 4),
                   executed_flops=exec_flops,
                   executed_mfma_frac=round(exec_flops / wall / 1e12 / BF16_PEAK_TFLOPS, 4)),
    )
    if not extras:
        return res

    # the same sweep with each chunk's routed reads replayed from one HIP graph
    if layers % sw.NSETS == 0:
        sw.capture_reads(layers)
        sw.sweep_graphed(layers, 2, batched)
        gwalls = []
        for _ in range(max(args.steps, 1)):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            sw.sweep_graphed(layers, chunks, batched)
            torch.cuda.synchronize()
            gwalls.append(time.perf_counter() - t0)
        gwall = statistics.mean(gwalls)
        res["graphed_reads"] = dict(
            value=round(tokens / gwall, 1), unit="tokens/s", ms_per_step=round(gwall * 1e3, 3),
            what="the same sweep, each chunk's L routed reads (router, row map, permute, "
                 "grouped APPLY, unpermute: the product API calls) captured once in a HIP "
                 "graph (torch.cuda.CUDAGraph) and replayed; updates and writes eager")
        sw.read_graph = None

    # stage totals of one sweep (events around the product calls)
    sw.marks = []
    sw.sweep(layers, chunks, batched)
    torch.cuda.synchronize()
    res["stages_ms_per_sweep"] = {k: round(v * 1e3, 2) for k, v in _stage_times(sw.marks).items()}
    sw.marks = None

    # per-kernel device time of one sweep, grouped by kernel symbol
    src = "torch.profiler device activity of one sweep"
    try:
        ktimes = kernel_times_profiled(lambda: sw.sweep(layers, chunks, batched))
    except Exception as exc:  # the tracer may be unavailable
        ktimes, src = None, f"profiler unavailable ({type(exc).__name__})"
    if ktimes is None:
        ktimes = kernel_times_from_profile(f"{key}_sweep.txt")
        src = f"committed rocprofv3 summary profiles/{key}_sweep.txt (older run)"
    tab = sw.launch_table(layers, chunks, batched)
    kern = {}
    for sym, (us, n) in sorted((ktimes or {}).items(), key=lambda kv: -kv[1][0]):
        d = dict(ms_per_sweep=round(us * 1e-3, 3), launches=n, avg_us=round(us / n, 2))
        if sym in tab:
            fl, by, _ = tab[sym]
            d.update(TFLOPs=round(fl / (us * 1e-6) / 1e12, 1),
                     mfma_frac=round(fl / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                     hbm_frac=round(by / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
        kern[sym] = d
        if len(kern) >= 14:
            break
    res["kernels_by_symbol"] = dict(source=src, top=kern)

    # roofline: the dominant kernel symbol by time per sweep
    dom = next((s for s in kern if s in tab), None)
    if dom is not None:
        fl, by, n = tab[dom]
        fl1, by1 = fl / n, by / n
        t_iso = sw.isolated(dom, batched)
        t_live = live.mean_s(dom)
        t_dom = (t_live if t_live is not None else
                 t_iso if t_iso is not None else kern[dom]["avg_us"] * 1e-6)
        ridge = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
        ai = fl1 / by1
        mfma = fl1 / t_dom / 1e12
        hbm = by1 / t_dom / 1e9
        common = dict(kernel=dom, avg_launch_us=round(t_dom * 1e6, 2),
                      timing=(live.describe(dom) if t_live is not None else
                              "HIP events around back-to-back launches on the launch stream"
                              if t_iso is not None else src),
                      isolated_launch_us=round(t_iso * 1e6, 2) if t_iso is not None else None,
                      launches_per_sweep=n, share_of_sweep=round(kern[dom]["ms_per_sweep"]
                                                                 * 1e-3 / wall, 4),
                      algorithmic_flops=int(fl1), algorithmic_bytes=int(by1),
                      arithmetic_intensity=round(ai, 1),
                      mfma_frac=round(mfma / BF16_PEAK_TFLOPS, 4),
                      hbm_frac=round(hbm / HBM_PEAK_GBS, 4),
                      traffic=_profile_traffic(f"{key}_sweep.txt", dom),
                      counter_mfma_util=_profile_value(f"{key}_sweep.txt", "mfma_util", dom))
        if ai >= ridge:
            res["roofline"] = dict(bound="mfma", achieved=round(mfma, 1), peak=BF16_PEAK_TFLOPS,
                                   unit="TFLOP/s", frac=round(mfma / BF16_PEAK_TFLOPS, 4), **common)
        else:
            res["roofline"] = dict(bound="hbm", achieved=round(hbm, 1), peak=HBM_PEAK_GBS,
                                   unit="GB/s", frac=round(hbm / HBM_PEAK_GBS, 4), **common)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_moe(sw, cfg, layers, chunks)
    return res


class LiveLaunchTimer:
    """HIP events on the launch stream around every call of the C-ABI entry
    points that launch exactly one kernel symbol, during the timed sweeps
    (the product code calls the library through uttt_amd._lib.call)."""

    def __init__(self, apply_symbols):
        # entry point -> the one kernel symbol it launches in the MoE sweep (the
        # weight gradients of the UPDATE forward; the APPLY's two products)
        gate, down = apply_symbols
        self.ENTRIES = {"uttt_grouped_wgrad_pair": "wg_kernel<false>",
                        "uttt_grouped_gate_up": gate, "uttt_grouped_gemm_nt": down}

    def __enter__(self):
        import torch

        from uttt_amd import _lib

        self._lib, self._orig, self.ev = _lib, _lib.call, {}

        def call(name, *args):
            sym = self.ENTRIES.get(name)
            if sym is None:
                return self._orig(name, *args)
            st = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            self._orig(name, *args)
            e1.record(st)
            self.ev.setdefault(sym, []).append((e0, e1))

        _lib.call = call
        return self

    def __exit__(self, *exc):
        self._lib.call = self._orig
        return False

    def mean_s(self, sym):
        evs = self.ev.get(sym)
        if not evs:
            return None
        import torch

        torch.cuda.synchronize()
        return statistics.mean(a.elapsed_time(b) for a, b in evs) * 1e-3

    def describe(self, sym):
        entry = next(k for k, v in self.ENTRIES.items() if v == sym)
        return (f"HIP events on the launch stream around each {entry} call of the timed sweeps "
                f"({len(self.ev[sym])} launches)")


def profile_kernel(args, key, name):
    """One short sweep to set up the pool and inputs of workload `key`, then
    only the isolated launch loop of kernel symbol `name` (for counter passes,
    which profile every launch)."""
    import torch

    cfg = MOE_CONFIGS[key]
    sw = MoeSweep(cfg, torch.device("cuda", 0))
    batched = args.update_schedule == "batched"
    sw.sweep(cfg["L"], 2, batched)
    torch.cuda.synchronize()
    t = sw.isolated(name, batched, reps=5)
    if t is None:
        raise SystemExit(f"bench.py: no isolated recipe for kernel {name!r}")
    return dict(workload=cfg["label"], kernel=name, us=round(t * 1e6, 2), launches=6)


def _median_time(fn, reps=3):
    """1 untimed warm-up run, then the median of `reps` timed runs (s)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline_moe(sw, cfg, layers, chunks):
    """The fp32 PyTorch restatement (oracle/fastweight.py, fp32 accumulation)
    of one layer-chunk's grouped APPLY, UPDATE (and UPDATE backward for the
    training slice) at the full shape, on all of this host's cores (1 warm-up
    run, median of 3); the sweep time is extrapolated as
    layers * (chunks * t_apply + (chunks-1) * t_update)."""
    import torch

    from oracle import fastweight as FW
    from uttt_amd import moe

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    st = sw.sets[0]
    with torch.no_grad():
        _, gs_a, _, _ = moe.route(st["x"], sw.R, sw.rcfg, routing_bias=sw.rbias)
        _, gs_u, _, _ = moe.route(st["k"], sw.R, sw.rcfg, routing_bias=sw.rbias)
    gs_a, gs_u = gs_a.cpu(), gs_u.cpu()
    W02, W1 = sw.W02.cpu(), sw.W1.cpu()
    g = torch.Generator().manual_seed(0)
    x, kk, vv = (torch.randn(1, sw.N, sw.D, generator=g).to(torch.bfloat16) for _ in range(3))
    lr = [torch.full((1, sw.N), 0.05).to(torch.bfloat16) for _ in range(3)]
    with FW.fp32_accumulate():
        t_apply = _median_time(lambda: FW.swiglu_ffn_fwd(W02, W1, x, gs_a))
        t_update = _median_time(lambda: FW.fast_weight_grads(W02, W1, kk, vv, *lr, gs_u))
        if cfg["train"]:
            GW02, GW1 = sw.GW02.cpu(), sw.GW1.cpu()
            t_update += _median_time(lambda: FW.fast_weight_grads_bwd(W02, W1, kk, vv, *lr, gs_u,
                                                                      GW02, GW1))
    t_sweep = layers * (chunks * t_apply + (chunks - 1) * t_update)
    return dict(value=round(SEQ / t_sweep, 2), unit="tokens/s", cores=cores,
                threads=torch.get_num_threads(), kind="port",
                sample=f"one layer-chunk at full shape (1 warm-up, median of 3): apply "
                       f"{t_apply:.2f} s, update{' fwd+bwd' if cfg['train'] else ''} "
                       f"{t_update:.2f} s (fp32 torch); sweep extrapolated x{layers} layers "
                       f"x{chunks} chunks",
                cpu=_cpu_model())


# ------------------------------------------------------------- dense sweep --
DENSE_CONFIGS = {
    # uTTT-Dense 124M shape, one shared fast weight, 12 layers
    "dense124m": dict(L=12, H=4, d=192, r=2, S=32768, chunk=2048,
                      label="uTTT-Dense 124M shared fast-weight apply+update (configs[1])"),
    # configs[0]'s single-layer shape, run on the GPU
    "dense_c0": dict(L=1, H=4, d=96, r=2, S=4096, chunk=512,
                     label="uTTT-Dense single layer, configs[0] shape, on the GPU"),
    # configs[1] as BASELINE words it: applied and updated sequentially per layer
    # per chunk (each layer writes right after its read; the reference's
    # uttt_dense supports only the aggregate schedule)
    "dense124m_chained": dict(L=12, H=4, d=192, r=2, S=32768, chunk=2048, schedule="chained",
                              label="uTTT-Dense 124M, chained schedule (configs[1] as worded)"),
    # configs[1] with the shipped write (uttt_llm/configs/main/124M/uttt_dense_r2.json:
    # use_momentum, use_moun): momentum + Newton-Schulz per d x d slice
    "dense124m_shipped": dict(L=12, H=4, d=192, r=2, S=32768, chunk=2048, shipped=True,
                              label="uTTT-Dense 124M (configs[1]) with the shipped write: "
                                    "momentum + Muon"),
}


def bench_dense(args, key):
    """One uTTT-Dense sweep: every layer reads every chunk with the chunk-start
    fast weights (grouped APPLY, one head = one batch), and every chunk but
    the last is written once from the layers' updates (aggregate mean: all
    layers' tokens in one grouped UPDATE per head, then the per-slice
    norm-preserving write).  Inputs: per layer q, k, v ~ N(0,1) L2-normalised
    per head, lr = sigmoid(N(0,1)) * 0.1; weights N(0, 1/sqrt(d))."""
    import torch

    from uttt_amd import dense as DN

    cfg = DENSE_CONFIGS[key]
    L_, H, d, r, S, c = cfg["L"], cfg["H"], cfg["d"], cfg["r"], cfg["S"], cfg["chunk"]
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    dh = r * d
    w = [torch.randn(*s, generator=g, device=dev) / d ** 0.5
         for s in ((1, H, dh, d), (1, H, d, dh), (1, H, dh, d))]
    nsets = min(L_, 4)
    sets = []
    for _ in range(nsets):
        qkv = [torch.nn.functional.normalize(torch.randn(1, S, H, d, generator=g, device=dev), dim=-1)
               .reshape(1, S, H * d).to(torch.bfloat16) for _ in range(3)]
        lr = torch.sigmoid(torch.randn(1, S, 3, generator=g, device=dev)) * 0.1
        sets.append(qkv + [lr])

    schedule = cfg.get("schedule", "aggregate")
    shipped = bool(cfg.get("shipped"))
    chunks = (S + c - 1) // c
    # per (chunk, layer) momentum coefficients (momentum_proj's sigmoid averaged
    # over the chunk's tokens), [b, 1, 1, 1]
    mcoef = torch.sigmoid(torch.randn(chunks, L_, 1, 1, 1, 1, generator=g, device=dev))

    def new_bank():
        return DN.SharedFastWeights(*w, r=r, use_momentum=shipped, use_moun=shipped)

    def sweep(bank, chunks):
        for ci in range(chunks):
            c0, c1 = ci * c, min(S, (ci + 1) * c)
            if schedule == "chained":   # each layer reads, then writes its own update
                for li in range(L_):
                    x = sets[li % nsets]
                    bank.read(x[0][:, c0:c1])
                    if ci < chunks - 1:
                        bank.write([x[1][:, c0:c1]], [x[2][:, c0:c1]], [x[3][:, c0:c1]],
                                   momentum_coeffs=[mcoef[ci, li]] if shipped else None)
                continue
            for li in range(L_):
                bank.read(sets[li % nsets][0][:, c0:c1])
            if ci < chunks - 1:
                st = [sets[li % nsets] for li in range(L_)]
                bank.write([x[1][:, c0:c1] for x in st], [x[2][:, c0:c1] for x in st],
                           [x[3][:, c0:c1] for x in st],
                           momentum_coeffs=list(mcoef[ci]) if shipped else None)

    for _ in range(max(args.warmup, 1)):
        sweep(new_bank(), min(chunks, 2))
    torch.cuda.synchronize()
    walls = []
    for _ in range(args.steps):
        bank = new_bank()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        sweep(bank, chunks)
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
    wall = statistics.mean(walls)
    # isolated timings (events around back-to-back calls on the stream)
    bank = new_bank()

    def timed(fn, reps=10):
        fn()
        e0, e1 = _events(2)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps

    q0 = sets[0][0][:, :c]
    t_read = timed(lambda: bank.read(q0))
    st = [sets[li % nsets] for li in range(L_)]
    t_write = timed(lambda: bank.write([x[1][:, :c] for x in st], [x[2][:, :c] for x in st],
                                       [x[3][:, :c] for x in st],
                                       momentum_coeffs=list(mcoef[0]) if shipped else None))
    nid = c * dh * d * H                                  # one layer-chunk, all heads
    sweep_flops = L_ * (chunks * 6 + (chunks - 1) * 12) * nid
    read_tf = 6 * nid / t_read / 1e12
    write_tf = 12 * L_ * nid / t_write / 1e12
    res = dict(
        metric="fast-weight apply+update tokens/s",
        value=round(S / wall, 1),
        unit="tokens/s",
        ms_per_step=round(wall * 1e3, 3),
        dtype="bf16",
        config={"workload": cfg["label"], "seq_len": S, "chunk": c, "layers": L_, "fw_heads": H,
                "head_dim": d, "fw_hidden": dh, "r": r,
                "schedule": ("aggregate (the reference's uttt_dense): all layers read the "
                             "chunk-start snapshot; one mean-reduced write per chunk"
                             if schedule == "aggregate" else
                             "chained: each layer reads the current weights, then writes its "
                             "own update (one write per layer per chunk)"),
                "write": "per-slice norm-preserving, norms from the bf16 fast weights"
                         + ("; momentum + Muon (Newton-Schulz per d x d slice)" if shipped
                            else "")},
        roofline=dict(bound="mfma", kernel="aggregate write (UPDATE over all layers + write)",
                      achieved=round(write_tf, 2), peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                      frac=round(write_tf / BF16_PEAK_TFLOPS, 4), traffic=None,
                      algorithmic_flops=12 * L_ * nid, avg_launch_us=round(t_write * 1e6, 2)),
        sweep=dict(algorithmic_flops=sweep_flops, TFLOPs=round(sweep_flops / wall / 1e12, 2),
                   mfma_frac=round(sweep_flops / wall / 1e12 / BF16_PEAK_TFLOPS, 4)),
        kernels={"read(one layer-chunk)": dict(us=round(t_read * 1e6, 2), TFLOPs=round(read_tf, 2)),
                 "write(one chunk, all layers)": dict(us=round(t_write * 1e6, 2),
                                                     TFLOPs=round(write_tf, 2))},
    )
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_dense(cfg, sets, w)
    return res


def cpu_baseline_dense(cfg, sets, w):
    """The fp32 PyTorch restatement (oracle/dense.py, fp32 accumulation) on this
    host's cores: configs[0]'s full single-layer sweep when L = 1, else one
    layer-chunk read and one layer's update at full shape, extrapolated to the
    sweep (L * (chunks reads + (chunks - 1) updates))."""
    import torch

    from oracle import dense as OD
    from oracle import fastweight as FW

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    L_, r, S, c = cfg["L"], cfg["r"], cfg["S"], cfg["chunk"]
    wc = [x.cpu() for x in w]
    fast = tuple(x.to(torch.bfloat16) for x in wc)
    q, k, v, lr = (x.cpu() for x in sets[0])
    chunks = (S + c - 1) // c
    with FW.fp32_accumulate():
        if L_ == 1:
            t0 = time.perf_counter()
            OD.sweep([q], [k], [v], [lr], fast, wc, r, c)
            t = time.perf_counter() - t0
            sample = f"full single-layer sweep ({chunks} chunks of {c})"
        else:
            t0 = time.perf_counter()
            OD.read(q[:, :c], *fast)
            t_read = time.perf_counter() - t0
            t0 = time.perf_counter()
            OD.compute_update(k[:, :c], v[:, :c], lr[:, :c], fast)
            t_upd = time.perf_counter() - t0
            t = L_ * (chunks * t_read + (chunks - 1) * t_upd)
            sample = (f"one layer-chunk: read {t_read:.3f} s, update {t_upd:.3f} s; sweep "
                      f"extrapolated x{L_} layers x{chunks} chunks")
    return dict(value=round(S / t, 2), unit="tokens/s", cores=cores, threads=threads, kind="port",
                sample=sample + f" (fp32 torch, {threads} threads)", cpu=_cpu_model())


# ---------------------------------------------------------- decode read --
def bench_decode(args):
    """Generation-time fast-weight read at the 760M shape: B = 8 sequences,
    each with its own expert pool (E=32, W0_W2 [6144, 1536], W1 [1536, 3072]),
    one new token per sequence through 24 layers.  A step = per layer, the
    fused router (shared router weights, Zipf(1.1) expert prior as selection
    bias, top-2, topk_renorm gates) and the decode read; value = tokens/s.
    The dominant cost is streaming each token's two experts' weights."""
    import torch

    from uttt_amd import _lib as L
    from uttt_amd import decode as DEC
    from uttt_amd.lact_moe_triton import lact_swiglu_ffn as SF
    from uttt_amd.lact_moe_triton import triton_permute as TP
    from uttt_amd.routing import route_tokens

    dev = torch.device("cuda", 0)
    B, T, E, k, D, I, layers = 8, 1, 32, 2, 1536, 3072, 24
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    W02 = (torch.randn(B, E, 2 * I, D, generator=g, device=dev) * D ** -0.5).to(bf)
    W1 = (torch.randn(B, E, D, I, generator=g, device=dev) * I ** -0.5).to(bf)
    xs = []
    for _ in range(layers):
        t = torch.randn(B, T, D, generator=g, device=dev)
        xs.append((t / (t.norm(dim=-1, keepdim=True) + 1e-5)).to(bf))
    R = torch.randn(E, D, generator=g, device=dev)
    rbias = -1.1 * torch.log(torch.arange(E, device=dev, dtype=torch.float32) + 1)
    routed = [None] * layers

    def step():
        for l in range(layers):
            mask, _, probs, _ = route_tokens(xs[l], R, k, combine_mode="topk_renorm",
                                             routing_bias=rbias)
            routed[l] = (mask, probs)
            DEC.moe_decode_read(xs[l], W02, W1, mask, probs, k)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_step = e0.elapsed_time(e1) * 1e-3 / args.steps

    # the read alone (two launches per call), back to back over the layers'
    # routings, and its algorithmic bytes: every selected (sequence, expert)
    # pair's W0_W2 and W1 once, plus x, the mask, the gates and the output
    reps = max(3, args.steps)
    nsel = sum(int(m.any(dim=2).sum().item()) for m, _ in routed)
    bytes_read = (nsel * 3 * I * D * 2 + layers * (2 * B * T * D * 2 + B * E * T * 5)) // layers
    e0.record()
    for _ in range(reps):
        for l in range(layers):
            DEC.moe_decode_read(xs[l], W02, W1, *routed[l], k)
    e1.record()
    torch.cuda.synchronize()
    t_read = e0.elapsed_time(e1) * 1e-3 / (reps * layers)

    # the same read through the grouped path (row map, permute, grouped
    # SwiGLU apply, unpermute), for comparison
    def grouped(l):
        mask, probs = routed[l]
        xp, _, rmap = TP.permute_with_expert_mask(xs[l], mask, probs, k)
        y = SF.grouped_swiglu_ffn_fwd(W02, W1, xp, mask.sum(-1).to(torch.int32))
        return TP.unpermute_and_merge_with_probs(y, rmap, probs)

    ref = grouped(0)
    ours = DEC.moe_decode_read(xs[0], W02, W1, *routed[0], k)
    err = (ours.float() - ref.float()).abs().max().item()
    assert err <= 2e-2 * ref.float().abs().max().item() + 1e-3, f"decode read diverged: {err}"
    e0.record()
    for _ in range(reps):
        for l in range(layers):
            grouped(l)
    e1.record()
    torch.cuda.synchronize()
    t_grouped = e0.elapsed_time(e1) * 1e-3 / (reps * layers)

    res = dict(
        metric="fast-weight decode read tokens/s (760M pool per sequence)",
        value=round(B * T / t_step, 1), unit="tokens/s",
        ms_per_step=round(t_step * 1e3, 4), wall_ms_per_step=round(wall / args.steps * 1e3, 4),
        dtype="bf16",
        config={"workload": "uTTT-MoE 760M decode read: router + routed SwiGLU read, 24 layers",
                "sequences": B, "tokens_per_step": T, "layers": layers, "experts": E, "topk": k,
                "d": D, "expert_hidden": I, "routing": "shared router, Zipf(1.1) selection bias"},
        roofline=dict(bound="hbm", kernel="moe_decode_read (gate/up + down launches)",
                      achieved=round(bytes_read / t_read / 1e9, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(bytes_read / t_read / 1e9 / HBM_PEAK_GBS, 4),
                      traffic=_profile_traffic("decode_read_760m.txt", "moe_decode_read"),
                      algorithmic_bytes=bytes_read, avg_call_us=round(t_read * 1e6, 2)),
        kernels={"decode read per layer": dict(us=round(t_read * 1e6, 2)),
                 "router per layer": dict(us=round((t_step / layers - t_read) * 1e6, 2),
                                          timing="step minus read"),
                 "grouped path per layer (row map, permute, apply, unpermute)":
                     dict(us=round(t_grouped * 1e6, 2))},
    )
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_decode(W02, W1, xs, routed, k, layers)
    return res


def cpu_baseline_decode(W02, W1, xs, routed, k, layers):
    """oracle/moe_read.apply_moe_grouped (fp32 torch: permute, grouped apply,
    unpermute) on this host's cores, layer by layer for about 10 s; the step
    is extrapolated to all layers."""
    import torch

    from oracle import moe_read as MR

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    B = xs[0].shape[0]
    t, done = 0.0, 0
    while t < 10.0 and done < layers:
        mask, probs = routed[done]
        for b in range(B):
            # only the sequence's selected experts travel to the host; their
            # ascending order keeps the merge's slot order
            sel = mask[b].any(dim=1).nonzero().flatten()
            x = xs[done][b:b + 1].cpu()
            w02, w1 = W02[b:b + 1, sel].cpu(), W1[b:b + 1, sel].cpu()
            m, p = mask[b:b + 1, sel].cpu(), probs[b:b + 1, sel].cpu()
            t0 = time.perf_counter()
            MR.apply_moe_grouped(x, w02, w1, m, p, k, fast=True)
            t += time.perf_counter() - t0
        done += 1
    per_layer = t / done
    return dict(value=round(B / (per_layer * layers), 2), unit="tokens/s", cores=cores,
                threads=threads,
                kind="port", sample=f"{done} of {layers} layers' reads in fp32 torch "
                                    f"({per_layer * 1e3:.0f} ms each, {threads} threads); "
                                    f"step extrapolated x{layers} layers", cpu=_cpu_model())


# ------------------------------------------------------------ Muon write --
def _ns5_flops(R, C):
    """Algorithmic FLOP of one Newton-Schulz5 of an R x C matrix (m = short
    side, n = long side): per iteration A = X X^T (2 m^2 n), A @ A (2 m^3),
    B @ X (2 m^2 n)."""
    m, n = min(R, C), max(R, C)
    return 5 * (4 * m * m * n + 2 * m ** 3)


def bench_muon(args):
    """The Muon write of one chunk on the 760M expert pool (E=32, W0/W2
    [3072, 1536], W1 [1536, 3072]; fp32 masters and momentum, bf16 gradients):
    momentum, Newton-Schulz5 per expert matrix, scaled add and the
    norm-preserving projection (modeling_recurrent_lact.py:754-825 with
    use_momentum and use_moun).  One step = the write of the three matrices;
    value = NS5 algorithmic TFLOP/s of the step."""
    import torch

    from uttt_amd import fast_weight_write as FWW

    dev = torch.device("cuda", 0)
    B, E, I, D = 1, 32, 3072, 1536
    g = torch.Generator().manual_seed(0)
    shapes = [(B, E, I, D), (B, E, D, I), (B, E, I, D)]
    masters = [(torch.randn(*s, generator=g) / D ** 0.5).to(dev) for s in shapes]
    grads = [(torch.randn(*s, generator=g) * 0.05).to(torch.bfloat16).to(dev) for s in shapes]
    moms = [(torch.randn(*s, generator=g) * 0.05).to(dev) for s in shapes]
    coeff = torch.full((B, 1, 1, 1), 0.9, device=dev)

    def step():
        return FWW.apply_moe_update_dense(tuple(grads), None, tuple(masters), tuple(moms), coeff,
                                          lr_scale=0.5, use_moun=True)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        out = step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_step = e0.elapsed_time(e1) * 1e-3 / args.steps
    flops = sum(B * E * _ns5_flops(*s[2:]) for s in shapes)

    # the NS5 chain of one matrix set alone (w0: 32 x [3072, 1536]), the
    # dominant part of the step, between events on its launch stream
    reps = max(3, args.steps)
    G0 = grads[0].reshape(B * E, I, D)
    FWW.newton_schulz5(G0, 0.5)
    e0.record()
    for _ in range(reps):
        FWW.newton_schulz5(G0, 0.5)
    e1.record()
    torch.cuda.synchronize()
    t_ns = e0.elapsed_time(e1) * 1e-3 / reps
    f_ns = B * E * _ns5_flops(I, D)

    # sanity: the write preserved the row norms of the masters
    m0 = masters[0].norm(dim=-1)
    m1 = out[1][0].norm(dim=-1)
    assert torch.allclose(m1, m0, rtol=1e-4), "Muon write broke the norm-preserving projection"
    res = dict(
        metric="Muon write NS5 TFLOP/s (760M expert pool, one chunk's write)",
        value=round(flops / t_step / 1e12, 2), unit="TFLOP/s",
        ms_per_step=round(t_step * 1e3, 3), wall_ms_per_step=round(wall / args.steps * 1e3, 3),
        dtype="bf16",
        config={"workload": "uTTT-MoE 760M pool write with momentum + Muon",
                "experts": E, "expert_hidden": I, "d": D,
                "step": "momentum, NS5 of 96 expert matrices, scaled add, norm-preserving write"},
        roofline=dict(bound="mfma", kernel="newton_schulz5 chain (w0: 32 x [3072,1536])",
                      achieved=round(f_ns / t_ns / 1e12, 1), peak=BF16_PEAK_TFLOPS,
                      unit="TFLOP/s", frac=round(f_ns / t_ns / 1e12 / BF16_PEAK_TFLOPS, 4),
                      traffic=None, algorithmic_flops=f_ns, avg_call_us=round(t_ns * 1e6, 1)),
        step_flops=flops, mfma_frac=round(flops / t_step / 1e12 / BF16_PEAK_TFLOPS, 4),
    )
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_muon(I, D)
    return res


def cpu_baseline_muon(I, D):
    """oracle/write.newton_schulz5 (bf16 CPU torch, the reference's
    arithmetic) on expert matrices of the pool (w0, w1, w2 in turn) until
    about 10 s have passed, on this host's cores."""
    import torch

    from oracle import write as OW

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    gen = torch.Generator().manual_seed(1)
    mats = [torch.randn(1, I, D, generator=gen), torch.randn(1, D, I, generator=gen)]
    done, flops, t = 0, 0, 0.0
    while t < 10.0 and done < 96:
        G = mats[done % 3 == 1]
        t0 = time.perf_counter()
        OW.newton_schulz5(G)
        t += time.perf_counter() - t0
        flops += _ns5_flops(I, D)
        done += 1
    return dict(value=round(flops / t / 1e12, 4), unit="TFLOP/s", cores=cores, threads=threads, kind="port",
                sample=f"NS5 of {done} of the 96 expert matrices ([{I}, {D}] / [{D}, {I}]) in "
                       f"bf16 torch: {t:.2f} s ({threads} threads)", cpu=_cpu_model())


def other_targets(args):
    """The other BASELINE targets measured in the same run: configs[2]
    permute / unpermute GB/s against HBM peak (and the C port of the step on
    one host core), the configs[3] uTTT-MoE 124M sweep, configs[4] with the
    shipped write (momentum + Muon), the uTTT-Dense sweeps of configs[1]
    (124M; aggregate, chained and with the shipped write) and configs[0]'s
    shape on the GPU, and configs[0] itself, the CPU fp32 reference sweep."""
    import copy

    cpu = not args.no_cpu_baseline
    a = copy.copy(args)
    a.no_cpu_baseline = not cpu      # configs[2]'s C port (about 10 s of CPU work)
    a.steps, a.warmup = 20, 5
    p = bench_permute(a)
    k = p["kernels"]
    a.no_cpu_baseline = True
    a.steps, a.warmup = 3, 1
    m = bench_moe(a, "moe124m", extras=True)
    a.steps, a.warmup = 2, 1
    ms = bench_moe(a, "moe760m_shipped", extras=False)
    a.steps, a.warmup = 3, 1
    d1 = bench_dense(a, "dense124m")
    d1c = bench_dense(a, "dense124m_chained")
    d1s = bench_dense(a, "dense124m_shipped")
    a.no_cpu_baseline = not cpu      # configs[0]: the full single-layer sweep on the CPU
    d0 = bench_dense(a, "dense_c0")
    dense = lambda r: dict(workload=r["config"]["workload"], value=r["value"], unit=r["unit"],
                           ms_per_step=r["ms_per_step"],
                           sweep_mfma_frac=r["sweep"]["mfma_frac"], kernels_us={
                               n: v["us"] for n, v in r["kernels"].items()},
                           roofline=r["roofline"])
    out = {
        "configs[2]_permute": dict(
            workload=p["config"]["workload"],
            permute_GBs=k["permute_chunk_kernel"]["GBs"],
            permute_hbm_frac=k["permute_chunk_kernel"]["hbm_frac"],
            unpermute_GBs=k["unpermute_chunk_kernel"]["GBs"],
            unpermute_hbm_frac=k["unpermute_chunk_kernel"]["hbm_frac"],
            step_GBs=p["value"], target_hbm_frac=0.70),
        "configs[3]_moe124m": dict(workload=m["config"]["workload"], value=m["value"],
                                   unit=m["unit"], ms_per_step=m["ms_per_step"],
                                   sweep_mfma_frac=m["sweep"]["mfma_frac"],
                                   graphed_reads=m.get("graphed_reads"),
                                   stages_ms_per_sweep=m.get("stages_ms_per_sweep"),
                                   top_kernels_us={
                                       k: v["avg_us"] for k, v in list(
                                           m.get("kernels_by_symbol", {}).get("top", {})
                                           .items())[:8]},
                                   roofline=m.get("roofline")),
        "configs[4]_shipped_write": dict(workload=ms["config"]["workload"], value=ms["value"],
                                         unit=ms["unit"], ms_per_step=ms["ms_per_step"]),
        "configs[1]_dense124m": dense(d1),
        "configs[1]_dense124m_chained": dense(d1c),
        "configs[1]_dense124m_shipped_write": dense(d1s),
        "configs[0]_dense_gpu": dense(d0),
    }
    if "permute_end_to_end" in p:
        out["configs[2]_permute"]["permute_with_expert_mask"] = p["permute_end_to_end"]
    if cpu:
        out["configs[2]_permute"]["cpu_port"] = p.get("cpu_baseline")
        out["configs[0]_cpu_reference"] = d0.get("cpu_baseline")
    return out


WORKLOADS = {"permute": bench_permute,
             "moe124m": lambda a: bench_moe(a, "moe124m"),
             "moe760m": lambda a: bench_moe(a, "moe760m"),
             "dense124m": lambda a: bench_dense(a, "dense124m"),
             "dense_c0": lambda a: bench_dense(a, "dense_c0"),
             "dense124m_chained": lambda a: bench_dense(a, "dense124m_chained"),
             "dense124m_shipped": lambda a: bench_dense(a, "dense124m_shipped"),
             "moe760m_shipped": lambda a: bench_moe(a, "moe760m_shipped"),
             "muon760m": bench_muon,
             "decode760m": bench_decode}
DEFAULT_WORKLOAD = "moe760m"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 20 for permute, 2 sweeps for the MoE workloads)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--update-schedule", default="batched", choices=["batched", "per-layer"],
                    help="MoE workloads: one grouped UPDATE per chunk over all writer layers "
                         "(batched) or one per writer (per-layer)")
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU baseline leg (profiling runs)")
    ap.add_argument("--no-extras", action="store_true",
                    help="default workload: skip the configs[2] / configs[3] measurements "
                         "that ride along in the line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one plain 256 MiB device copy (PMC scaling)")
    ap.add_argument("--profile-kernel", default=None,
                    help="MoE workloads: set up one sweep's state, then only run the isolated "
                         "launch loop of this kernel (e.g. gate_up, down_proj, wgrad) and print "
                         "its mean launch time; for rocprofv3 counter passes")
    args = ap.parse_args()
    moe = args.workload.startswith(("moe", "dense"))
    if args.steps is None:
        args.steps = 2 if moe else 20
    if args.warmup is None:
        args.warmup = 1 if moe else 5
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part of it "
              "(use --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    from uttt_amd import _lib as L

    L.lib()  # fail loudly if the HIP library is not built
    if args.copy_calibration:
        copy_calibration()
    if args.profile_kernel:
        if not args.workload.startswith("moe"):
            print("bench.py: --profile-kernel applies to the MoE workloads", file=sys.stderr)
            sys.exit(2)
        print(json.dumps(profile_kernel(args, args.workload, args.profile_kernel)), flush=True)
        return
    res = WORKLOADS[args.workload](args)
    if args.workload == DEFAULT_WORKLOAD and not args.no_extras:
        res["other_targets"] = other_targets(args)
    line = dict(metric=res.pop("metric"), value=res.pop("value"), unit=res.pop("unit"),
                n_gpus=1, steps=args.steps, warmup=args.warmup,
                ms_per_step=res.pop("ms_per_step"), higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype=res.pop("dtype"), data="synthetic (seeded)",
                config=res.pop("config"))
    line.update(res)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
