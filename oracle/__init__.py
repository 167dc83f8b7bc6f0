"""CPU oracle of uTTT's fast-weight hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped.  The product package `uttt_amd` never
imports it.

Contents (each function cites the reference file:line it restates):
  permute     - row map / permute / unpermute / permute_kv_and_lrs, restated
                in C (permute_oracle.c, built by build.py) and the backward
                passes in fp32 torch;
  routing     - create_router_mask_sizes_probs and the router logits;
  fastweight  - grouped SwiGLU apply, the dot-product-loss update and its
                backward, fp32 torch with the reference's bf16 rounding points;
  write       - the norm-preserving write of the MoE pool and of the dense
                shared state, with momentum and the Newton-Schulz5 (Muon) step;
  moe_read    - the routed read (permute, grouped apply, gate-weighted
                unpermute) composed from the pieces above;
  dense       - the uTTT-Dense / LaCT single-layer chunk loop.

Every function is pinned by a check that a plausible mistake would fail
(golden vectors, invariants, autograd, closed forms, brute force, planted
mistakes); the checks are the tests/test_oracle_*.py files.
"""
