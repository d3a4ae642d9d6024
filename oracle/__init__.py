"""The oracle: a CPU restatement of Difflet's reference math for the DiT denoise step.

TEST INFRASTRUCTURE ONLY. Nothing in the product (difflet_amd/) imports, calls or links this
package; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
the checker or as the timed CPU baseline, never as the thing measured or shipped.

Modules:
  ops   -- the `cpu` backend ops (attention, RMSNorm laws, RoPE laws, LayerNorm/adaLN, GELU,
           linear, timestep embedding, FLUX RoPE tables), fp32 torch on the CPU.
  mx    -- the MXFP8 block law (difflet/quant/mx.py) and an e4m3fn encoder, numpy integer math.
  fp8   -- the per-row e4m3 law of the per-channel x per-token fp8 linear (no reference
           counterpart; the law is this build's, fixed in include/difflet_rocm.h).
  flux  -- FLUX.1 double/single blocks and the full transformer forward, seeded random weights.

Each function cites the reference file:line it restates. Pins (what checks each function
against something other than itself) live in tests/test_oracle_*.py.
"""
