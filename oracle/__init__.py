"""CPU oracle of uTTT's fast-weight hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped.  The product package `uttt_amd` never
imports it.

Contents (each function cites the reference file:line it restates):
  permute     - row map / permute / unpermute / permute_kv_and_lrs, restated
                in C (permute_oracle.c, built by build.py) and the backward
                passes in fp32 torch;
  routing     - create_router_mask_sizes_probs in fp32 torch;
  fastweight  - grouped SwiGLU apply, the dot-product-loss update, its
                backward and the norm-preserving write, fp32 torch with the
                reference's bf16 rounding points;
  dense       - the uTTT-Dense / LaCT single-layer chunk loop.

How each function is pinned (golden vectors, invariants, autograd, brute
force) is listed in tests/ and summarised in DESIGN.md's parity table.
"""
