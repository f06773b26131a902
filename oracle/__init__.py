"""CPU oracle for the fake-quant attention path.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes for
``low_bit_fake_quant.fake_quant_attention`` so that the HIP product can be
checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker /
reported CPU baseline -- never as a code path of the product.

Modules and the reference code each one follows (paths relative to the
reference checkout):

* ``fp8``        -- OCP E4M3FN encode/decode (RNE), the format behind
                    ``torch.float8_e4m3fn`` / Triton ``float8e4nv``.
* ``quant``      -- ``quant_triton.py:26-416`` (block / channel / MX quant and
                    dequant).
* ``preprocess`` -- ``preprocess.py:10-193`` (K smoothing, grouped Q mean, V
                    per-block mean) with a fixed fp64 summation order.
* ``hadamard``   -- ``hadamard.py:25-117`` (random signs + torch FWHT).
* ``kmeans``     -- ``kmeans.py:44-135`` (reorder plumbing); the clustering
                    itself follows this project's own deterministic Lloyd
                    specification (flash-kmeans is not available).
* ``attention``  -- ``attention_triton.py:109-407`` (streaming K-loop:
                    qm correction, online / qm_k row max, P quant, V kinds,
                    V-smoothing accumulator, BLASST skip/fill) and
                    ``attention.py:366-395`` (qm_k row-max estimate).
* ``pipeline``   -- ``attention.py:166-321, 505-806`` (preprocess order,
                    SDPA path, P-requant marshalling, inverse Q gather).

Pinning status of every function is listed in each module header.
"""
