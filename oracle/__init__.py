"""CPU oracle for SAF3R head-wise sparse global attention.

TEST INFRASTRUCTURE ONLY. This package restates the reference algorithm on the CPU so
that the HIP kernels can be checked against it. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it,
and only to check results (or, for ``cpu_baseline``, as the timed CPU restatement). The
product package never imports it and has no CPU fallback.

Modules
-------
selection   ctypes binding of ``selection.c`` (sortable key, block pooling, block scores,
            per-frame / global top-k): integer-exact, fully specified fp32 order.
attention   torch fp32/fp64 restatement of the attention patterns (dense, frame-local,
            anchor+local, block-dynamic, token-dynamic, anchor-only), the gather
            attention, RoPE-2D, QK-LayerNorm and the patched layer forward.
"""
