"""akv_amd: MI355X-native (gfx950) Drop + Reposition of retained KV.

A drop-in for the KV-cache hot path of thu-nics/AKV:

* ``akv_amd.ops.reposition_kv_layers`` -- fused all-layer K re-rotation and
  K-tail / V move (HIP kernel, bit-exact with the reference arithmetic);
* ``akv_amd.tables.compact_rows`` -- batched page-table compaction: terminal
  request rows, freed slots, copy lists, decode layout and compacted rows;
* ``akv_amd.page_table`` -- decode indices, window lengths, indptr rebuild
  over the reference registry's rows, and the side-row / extend writes of
  request rows;
* ``akv_amd.context_attention.extend_attention_fwd`` -- prefill attention
  over the compacted rows with context positions;
* ``akv_amd.plan.compile_context_layout`` -- the host event compiler;
* ``akv_amd.occurrence`` / ``akv_amd.ownership`` -- the prefill's occurrence
  window and slot ownership across forwards;
* ``akv_amd.transfer.copy_kv_rows`` -- K/V row copies of the P -> D handoff.

The reference's host classes (model binding, decode registry, prefill
metadata, P -> D transfer planning, the request row store) stay the callers:
each calls these functions where it called a Triton kernel or a numpy
planner, with the same arguments.

All device work is in ``libakv_amd.so`` (C ABI: ``include/akv_amd.h``),
built by ``python -m akv_amd.build``.  There is no CPU fallback.
"""

__version__ = "0.1.0"
