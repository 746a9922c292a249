"""Parity oracle for the three fused ops -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the timed CPU restatement).  The product path
(``nuvla_forge_amd``) never imports, calls or falls back to it.

Modules:
  numerics   NumPy restatement (fp64 by default) of the reference math with
             analytic backward passes -- the checker the GPU parity tests use.
  torch_cpu  PyTorch-CPU restatement of the reference's eager path
             (``kernels/reference.py`` + the row-chunk CE loop), forward plus
             autograd backward -- the CPU baseline ``bench.py`` times.

How each function is pinned (tests/test_oracle.py):
  adaln_forward / adaln_backward    fp64 central differences of the forward for
      all six gradients; torch fp64 autograd of the torch_cpu restatement;
      hand-computed known answers; gate=0 => h == x exactly; w=1, s=sh=0 =>
      rms(out) = 1; shift enters out additively; golden fixtures.
  swiglu_forward / swiglu_backward  central differences; torch fp64 autograd
      of F.silu; closed-form values at a = 0 and saturation; golden fixtures.
  ce_forward_backward               central differences (loss vs dH, dW);
      torch fp64 F.cross_entropy + autograd; brute-force per-row loop on tiny
      inputs; all-ignored => loss 0 and zero grads; ignored rows carry zero
      dH; the mean uses the valid count; golden fixtures.
No oracle function is left without such a check ("parity unpinned": none).
"""
