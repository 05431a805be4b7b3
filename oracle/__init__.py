"""CPU oracle for the LATENT fused low-rank expert FFN.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`latent_amd`) may
import, call or link anything under `oracle/`. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and
there only to check results, never as the thing measured or shipped.

Contents:
  latent_ref   numpy restatement of the reference codec (NF4 / INT8), CPU
               runtime (`swiglu_expert`), stacked-factor layout, the per-group
               INT8 extension and a layer-level router-weighted MoE forward.
  routing      numpy restatement of the routing front-ends used by the
               synthetic workloads (softmax top-k, Zipf skew, adaptive drop).
  synth        seeded generators of small layers, and the load-time
               factorization (randomized_svd, choose_rank, make_factors of
               loader/latent_loader.py:66-108).
"""
