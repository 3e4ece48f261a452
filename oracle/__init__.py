"""CPU oracle for the Drop + Reposition hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path
that the HIP library replaces, to check it: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product (``akv_amd``) never imports, links or calls anything
here, and it has no CPU fallback: when the HIP library is missing it raises.

Modules and the reference code each one restates (paths relative to the
reference repository root):

``bf16``        IEEE round-to-nearest-even fp32 -> bf16/fp16 packing used by
                every store of the Reposition kernel (Triton's default
                downcast, ``context_reposition.py:103-112``).
``reposition``  ``_reposition_layers_kernel`` op order
                (``akv/system/sglang/kernels/ops/attention/context_reposition.py:54-123``)
                and the wrapper's validation (``:126-236``).
``cpu_torch``   the same Reposition arithmetic as torch CPU tensor operations
                over every host thread: the CPU baseline that ``bench.py``
                times, pinned bit for bit to ``reposition``.
``events``      the linked-list Drop/Reposition replay of
                ``akv/system/sglang/kernels/ops/attention/context_plan.py:80-532``
                and its driver ``akv/system/sglang/srt/context_system/ir.py:113-274``.
``occurrence``  the final-forward ownership result of
                ``akv/system/sglang/srt/context_system/occurrence.py:112-265,341-466,632-767``
                (terminal row, retired slots, copy lists, decode layout).
``decode``      ``context_decode_indices`` / ``context_window_lengths``
                (``akv/system/sglang/kernels/ops/attention/context_page_table.py:7-76``),
                ``write_row_slots`` (``.../ops/memory/context_rows.py:7-15``) and the
                ``kv_indptr = cumsum`` rebuild (``akv/system/sglang.patch:2266-2268``).
``attention``   one GQA decode step with attention sinks, the consumer of the
                compacted metadata (sink normalisation of
                ``akv/system/sglang/srt/layers/attention/context_backend.py:254-272``).
``ownership``   request-local page ownership across prefill forwards (chunked
                prefill, borrowed prefixes, recovery gaps, publication):
                ``plan_occurrence_materialization`` and ``OccurrenceState``
                (``akv/system/sglang/srt/context_system/occurrence.py:341-920``).
``paging``      page-granular Drop + Reposition with copy-on-write; the
                reference rejects page sizes other than 1
                (``context_reposition.py:153-154``), so this module is the
                extension's specification, pinned to ``occurrence`` at page size 1.

How each function is pinned (golden vectors / closed forms / brute force /
invariants) is stated in its module docstring.  The RoPE tables are not part
of the oracle: the kernel and the oracle read the same table, so parity of
the kernel holds for any table.
"""
