#!/usr/bin/env python3
"""Benchmark of uTTT's fast-weight hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line (rank 0).  Workloads (seeded synthetic inputs, resident
in HBM before the timed region starts):

  permute   token permute + gate-weighted unpermute by expert, T=65536, E=16,
            top-2, payload bf16 [T, 768]; one step = row map + permute +
            unpermute of one batch; value = algorithmic GB/s of the step.

Timing: W untimed steps, then K steps bracketed by torch.cuda.synchronize();
per-kernel durations come from HIP events recorded on the stream the kernels
are launched on (torch's current stream, which the C-ABI calls receive).
`roofline` reports the dominant kernel against MI355X's published peak;
`cpu_baseline` times the CPU restatement under oracle/ on this host's cores
(rank 0, N=1) on a bounded sample of the same workload.

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

    def step(s, ev=None):
        p = s["gates"]
        if ev is not None:
            ev[0].record()
        L.call("uttt_make_row_id_map", L.ptr(s["mask"]), 1, s["mask"].stride(0),
               s["mask"].stride(1), s["mask"].stride(2), B, T, E, L.ptr(s["rmap"]),
               L.ptr(s["gs"]), L.ptr(ws), ws_bytes, stream)
        if ev is not None:
            ev[1].record()
        L.call("uttt_permute_fwd", L.ptr(s["x"]), BF16, B, T, D, L.ptr(s["rmap"]), E,
               L.ptr(p), p.stride(0), p.stride(1), p.stride(2), L.ptr(s["xp"]), k * T,
               L.ptr(s["pp"]), stream)
        if ev is not None:
            ev[2].record()
        L.call("uttt_unpermute_fwd", L.ptr(s["xp"]), BF16, B, k * T, D, L.ptr(s["rmap"]), T, E,
               L.ptr(p), p.stride(0), p.stride(1), p.stride(2), L.ptr(s["y"]), stream)
        if ev is not None:
            ev[3].record()

    for i in range(args.warmup):
        step(sets[i % nsets])
    torch.cuda.synchronize()
    evs = [_events(4) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(sets[i % nsets], evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_map = [e[0].elapsed_time(e[1]) * 1e-3 for e in evs]
    t_perm = [e[1].elapsed_time(e[2]) * 1e-3 for e in evs]
    t_unp = [e[2].elapsed_time(e[3]) * 1e-3 for e in evs]

    # algorithmic bytes (each tensor once): permute reads x and the k row ids
    # per token and writes k copies; unpermute reads the k rows, their gates
    # and row ids, and writes one row per token.
    row = D * 2
    perm_bytes = T * row + k * T * 4 + k * T * row
    unp_bytes = k * T * row + k * T * (4 + 4) + T * row
    map_bytes = E * T * 1 + T * (2 * E + 1) * 4
    step_bytes = perm_bytes + unp_bytes
    t_p = statistics.mean(t_perm)
    t_u = statistics.mean(t_unp)
    value = step_bytes / (t_p + t_u) / 1e9

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
        ms_per_step=round(wall / args.steps * 1e3, 4),
        dtype="bf16",
        config={"workload": "uttt-moe permute/unpermute microbench (configs[2])", "T": T, "E": E,
                "topk": k, "hidden": D, "payload": "bf16", "buffer_sets": nsets},
        roofline=dict(
            bound="hbm", kernel="permute_fwd_kernel",
            achieved=round(perm_bytes / t_p / 1e9, 2), peak=HBM_PEAK_GBS, unit="GB/s",
            frac=round(perm_bytes / t_p / 1e9 / HBM_PEAK_GBS, 4), traffic=None,
            algorithmic_bytes=perm_bytes, avg_launch_us=round(t_p * 1e6, 3),
        ),
        kernels={
            "row_id_map(3 launches)": dict(us=round(statistics.mean(t_map) * 1e6, 3),
                                           GBs=round(map_bytes / statistics.mean(t_map) / 1e9, 1)),
            "permute_fwd_kernel": dict(us=round(t_p * 1e6, 3), GBs=round(perm_bytes / t_p / 1e9, 1),
                                       hbm_frac=round(perm_bytes / t_p / 1e9 / HBM_PEAK_GBS, 4)),
            "unpermute_fwd_kernel": dict(us=round(t_u * 1e6, 3),
                                         GBs=round(unp_bytes / t_u / 1e9, 1),
                                         hbm_frac=round(unp_bytes / t_u / 1e9 / HBM_PEAK_GBS, 4)),
        },
    )
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_permute(sets[0], B, T, E, k, D, step_bytes)
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


WORKLOADS = {"permute": bench_permute}
DEFAULT_WORKLOAD = "permute"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU baseline leg (profiling runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one plain 256 MiB device copy (PMC scaling)")
    args = ap.parse_args()
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
    res = WORKLOADS[args.workload](args)
    line = dict(metric=res.pop("metric"), value=res.pop("value"), unit=res.pop("unit"),
                n_gpus=1, steps=args.steps, warmup=args.warmup,
                ms_per_step=res.pop("ms_per_step"), higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype=res.pop("dtype"), data="synthetic (seeded)",
                config=res.pop("config"))
    line.update(res)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
