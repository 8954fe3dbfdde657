"""CPU oracle for the DP-SGD clip + noise path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of
JetBrains-Research/opaque for per-example clipping, AUTO-S scaling, per-group
clipping, the batch sum and the Gaussian noise sampler, plus a restatement of
the device Philox4x32-10 stream.  It is the checker the GPU path is compared
against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
``opaque_amd`` never does.

Modules and what pins them (paths relative to the reference's packages/):

* ``dp_ref``     clip_pytree / auto_scale_pytree / per-group / clipped_grad /
                 gaussian_noise restated from opaque-engine/.../clipping/
                 _pytree.py, _clipped_fun.py, _clipped_grad.py, _auto.py,
                 _per_group.py and opaque-dpsgd/.../noise/_gaussian.py.
                 Pinned by the reference tests' known answers (per-group
                 0.6/0.8/3.0, sqrt(194), 50; AUTO-S 1/(5+0.01) etc.; the
                 clipped_grad doc example losses [4.5, 8, 12.5] and norms
                 [3, 4, 5]; global_norm 13; per-group sigma 4.0 and
                 6.928203230275509), by invariants (bound holds as stored,
                 exact passthrough, C=0 gives zeros) and by brute force
                 (per-example loops against vmap).
* ``lora_ref``   per-example LoRA factor gradients and full-weight gradient
                 norms (opaque-patches/.../kernels/lora.py:164-176), in fp64;
                 pinned against autograd on single examples and against the
                 Gram identity ||G^T X||_F^2 = sum_{t,s}(g_t.g_s)(x_t.x_s).
* ``philox_ref`` Philox4x32-10 (Salmon et al., SC 2011) in numpy and the
                 device noise transform in fp64; pinned by the Random123
                 known-answer vectors.

Parity status: the exact mt19937 noise values of the reference are not
reproduced by the device path (which draws from Philox); noise parity is
distributional (mean, variance, KS) and determinism, as the reference's own
tests check it.  The guard constants and clip arithmetic are restated from
source; no reference test pins their float sequence op for op, so they are
cross-checked by the invariants above.
"""
