"""CPU oracle for the cached block-diffusion step.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on its hot path:

* ``oracle.model``      -- the nine entry points of ``fast_dllm_relax/model/cuda.py`` (numpy, with an
                           exact emulation of the bf16 / fp16 rounding points of the reference's
                           precision order, or plain fp32).
* ``oracle.runtime``    -- the prefix-cache contract and the decode loop of
                           ``fast_dllm_relax/runtime.py`` driven by ``oracle.model``.
* ``oracle/confidence.c`` (loaded through ``oracle.confidence``) -- the per-row argmax / max-softmax
                           confidence and the 0.9-threshold unmask rule, with the reduction order
                           and the exp the HIP kernels use, so identical logits give identical bits.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it,
and only as the checker.  The product (``fast-dllm-relax_amd``) never imports, links or runs it; the
product fails loudly when its HIP library is missing instead of falling back to anything here.

Pinning (what checks this oracle independently of its own formulas) is listed per function in the
module docstrings and exercised by ``tests/test_oracle_pinning.py``.
"""
