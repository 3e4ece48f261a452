"""Engine-lifetime layer bindings of the Context prefill.

Mirror of ``akv/system/sglang/srt/layers/attention/context_backend.py``:
``ContextForwardMetadata`` (``:345-358``), ``ContextPoolLayer``
(``:361-370``), ``ContextModelBinding`` (``:373-529``) and
``ContextPrefillInput`` (``:532-663``), with the same constructor
arguments, validation and messages.  The model, KV pool and index
translator are the engine's own objects, read through the attributes the
reference reads (``model.modules()`` with ``attn`` / ``rotary_emb``,
``pool.get_kv_buffer(layer_id)``, ``translator.translate_full_attn_ids`` /
``sliding_window_write_loc_for``).  Every KV move is
``reposition_kv_layers`` (HIP); compatible layers share one launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .context_attention import ContextAttentionMetadata, ContextAttentionPlan, ContextSequence
from .ops import ContextLayerCopy, reposition_kv_layers
from .request_rows import request_row


@dataclass(frozen=True)
class ContextForwardMetadata:
    """Bound attention metadata (full and sliding-window pools) and each
    layer's copy-on-write, keyed by global layer id."""

    full: ContextAttentionMetadata
    sliding_window: ContextAttentionMetadata | None
    layer_copies: dict

    def for_layer(self, layer) -> ContextAttentionMetadata:
        if layer.sliding_window_size is not None and layer.sliding_window_size > -1:
            if self.sliding_window is None:
                raise ValueError("Context SWA metadata was not bound")
            return self.sliding_window
        return self.full


@dataclass(frozen=True)
class ContextPoolLayer:
    layer_id: int
    sliding_window: bool
    k_ptr: torch.Tensor
    v_ptr: torch.Tensor
    k_buffer: torch.Tensor
    v_buffer: torch.Tensor
    cos_sin_cache: torch.Tensor
    is_neox_style: bool
    rotary_dim: int


class ContextModelBinding:
    """Per-layer KV buffers and RoPE tables of the model, bound once.

    ``reposition_existing`` moves completed versions of every layer, one
    launch per group of layers that share (window kind, shape, strides,
    dtype, table, style, rotary width); ``bind`` turns a prefill input into
    the per-layer metadata of one forward.
    """

    def __init__(self, model, pool, translator, *, page_size: int):
        if page_size != 1:
            raise ValueError("Context model binding requires page_size=1")
        layers = []
        for module in model.modules():
            attn = getattr(module, "attn", None)
            rotary = getattr(module, "rotary_emb", None)
            if attn is None or rotary is None or not hasattr(attn, "layer_id"):
                continue
            k, v = pool.get_kv_buffer(attn.layer_id)
            table = getattr(rotary, "cos_sin_cache", None)
            rotary_dim = getattr(rotary, "rotary_dim", k.shape[-1])
            if (
                k.ndim != 3
                or v.shape != k.shape
                or k.dtype not in (torch.float16, torch.bfloat16)
                or v.dtype != k.dtype
                or table is None
                or table.ndim != 2
                or type(rotary_dim) is not int
                or not 0 < rotary_dim <= k.shape[-1]
                or rotary_dim % 2
                or table.shape[1] != rotary_dim
                or k.device != v.device
                or k.device != table.device
                or k.stride(-1) != 1
                or v.stride(-1) != 1
            ):
                raise ValueError("Context needs native NHD KV and valid native rotary_dim")
            window = attn.sliding_window_size
            layers.append(ContextPoolLayer(
                attn.layer_id, window is not None and window > -1,
                torch.tensor([k.data_ptr()], dtype=torch.uint64, device=k.device),
                torch.tensor([v.data_ptr()], dtype=torch.uint64, device=v.device),
                k, v, table, rotary.is_neox_style, rotary_dim))
        if not layers or len({layer.layer_id for layer in layers}) != len(layers):
            raise ValueError("Context model must expose unique native attention layers")
        self.layers = tuple(layers)
        self.translator = translator
        self.has_swa = any(layer.sliding_window for layer in layers)
        self._groups = None

    def _copy_groups(self):
        if self._groups is None:
            groups = {}
            for layer in self.layers:
                key = (layer.sliding_window, tuple(layer.k_buffer.shape), layer.k_buffer.stride(),
                       layer.v_buffer.stride(), layer.k_buffer.dtype, layer.cos_sin_cache.data_ptr(),
                       layer.is_neox_style, layer.rotary_dim)
                groups.setdefault(key, []).append(layer)
            self._groups = tuple((items[0], torch.cat([x.k_ptr for x in items]), torch.cat([x.v_ptr for x in items]))
                                 for items in groups.values())
        return self._groups

    @property
    def launches(self):
        """Reposition launches of one ``reposition_existing``."""
        return len(self._copy_groups())

    def reposition_existing(self, source, destination, positions):
        """Move completed versions of every layer (no per-layer birth
        dependency): one launch per group of compatible layers."""
        source = self.translator.translate_full_attn_ids(source).to(torch.int32)
        destination = self.translator.translate_full_attn_ids(destination).to(torch.int32)
        for layer, k_ptrs, v_ptrs in self._copy_groups():
            src, dst, separate_swa = source, destination, False
            if layer.sliding_window:
                swa_src = self.translator.sliding_window_write_loc_for(source)
                if swa_src is not None:
                    separate_swa = True
                    src = swa_src.to(torch.int32)
                    dst = self.translator.sliding_window_write_loc_for(destination).to(torch.int32)
            reposition_kv_layers(k_ptrs, v_ptrs, layer.k_buffer, layer.v_buffer, src, dst, positions,
                                 layer.cos_sin_cache, is_neox_style=layer.is_neox_style,
                                 rotary_dim=layer.rotary_dim, skip_unmapped=separate_swa)

    def bind(self, inputs: ContextPrefillInput) -> ContextForwardMetadata:
        """Physical slots of the forward's occurrences and copies, in the
        full pool and (when separate) the sliding-window pool."""
        full_slots = self.translator.translate_full_attn_ids(inputs.occurrence_slots.clamp(min=0))
        copy_source = self.translator.translate_full_attn_ids(inputs.copy_sources)
        copy_destination = self.translator.translate_full_attn_ids(inputs.copy_destinations)
        full = inputs.attention_plan.bind(full_slots)
        swa = None
        separate_swa_pool = False
        swa_source, swa_destination = copy_source, copy_destination
        if self.has_swa:
            swa_slots = self.translator.sliding_window_write_loc_for(full_slots)
            if swa_slots is None:
                swa = full  # SWA layers share the full pool's slot space
            else:
                separate_swa_pool = True
                swa_source = self.translator.sliding_window_write_loc_for(copy_source)
                swa_destination = self.translator.sliding_window_write_loc_for(copy_destination)
                if swa_source is None or swa_destination is None:
                    raise ValueError("Context SWA pool is missing its native index mapping")
                swa = inputs.attention_plan.bind(swa_slots)
        copies = {}
        if len(inputs.copy_sources):
            for layer in self.layers:
                src = swa_source if layer.sliding_window else copy_source
                dst = swa_destination if layer.sliding_window else copy_destination
                copies[layer.layer_id] = ContextLayerCopy(
                    layer.k_ptr, layer.v_ptr, layer.k_buffer, layer.v_buffer, src.to(torch.int32),
                    dst.to(torch.int32), inputs.copy_positions, layer.cos_sin_cache, layer.is_neox_style,
                    skip_unmapped=layer.sliding_window and separate_swa_pool, rotary_dim=layer.rotary_dim)
        return ContextForwardMetadata(full, swa, copies)


@dataclass(frozen=True)
class ContextPrefillInput:
    """Immutable forward snapshot; its pages stay leased until completion."""

    attention_plan: ContextAttentionPlan
    occurrence_slots: torch.Tensor
    copy_sources: torch.Tensor
    copy_destinations: torch.Tensor
    copy_positions: torch.Tensor
    model_binding: ContextModelBinding | None

    @classmethod
    def from_prepared_batch(cls, batch, *, decode: bool):
        """Wrap native rows when an ordinary prefill mixes with Context
        decode: ordinary requests read their whole row, a Context decode
        reads its compacted prompt plus its generated tail."""
        from .page_table import ContextDecodeLayout

        sequences, slots = [], []
        for i, (req, raw_len) in enumerate(zip(batch.reqs, batch.seq_lens_cpu.tolist())):
            query_len = 1 if decode else batch.extend_lens[i]
            row = request_row(batch.req_to_token_pool, req.kv.req_pool_idx)[:raw_len]
            if req.context_program is None:
                sequences.append(ContextSequence.ordinary(raw_len - query_len, query_len))
                slots.append(row)
                continue
            if not decode:
                raise ValueError("Context prefill must use its admitted occurrence plan")
            view = req.context_decode_layout
            if view is None:
                view = ContextDecodeLayout.from_layout(req.context_program.layout, row.device)
                req.context_decode_layout = view
            generated = raw_len - view.prompt_length
            if generated < 1:
                raise ValueError("Mixed Context decode requires its native allocated query")
            raw = np.concatenate((view.raw_indices, np.arange(view.prompt_length, raw_len)))
            positions = np.concatenate((view.positions, np.arange(view.next_position,
                                                                  view.next_position + generated)))
            n = len(raw)
            sequences.append(ContextSequence(n, (1,), np.asarray([0, n - 1], dtype=np.int64),
                                             np.arange(n - 1, dtype=np.int64), positions[-1:].astype(np.int64),
                                             positions[:-1].astype(np.int64)))
            slots.append(row[torch.from_numpy(raw.astype(np.int64)).to(row.device, non_blocking=True)])
        empty = batch.out_cache_loc[:0].to(torch.int32)
        return cls(ContextAttentionPlan.merge(sequences), torch.cat(slots), empty, empty, empty.reshape(0, 2), None)

    @classmethod
    def concatenate(cls, inputs):
        sequences = []
        for item in inputs:
            plan = item.attention_plan
            _, offsets, occurrences, query_positions, prefix_positions = (
                plan.packed[a:b].numpy() for a, b in plan.field_ranges)
            sequences.append(ContextSequence(plan.occurrence_count, plan.query_lengths, offsets, occurrences,
                                             query_positions, prefix_positions))
        return cls(
            ContextAttentionPlan.merge(sequences),
            torch.cat([item.occurrence_slots for item in inputs]),
            torch.cat([item.copy_sources for item in inputs]),
            torch.cat([item.copy_destinations for item in inputs]),
            torch.cat([item.copy_positions for item in inputs]),
            None,
        )

    def bind(self, model_runner=None) -> ContextForwardMetadata:
        if (
            self.copy_sources.ndim != 1
            or self.copy_destinations.shape != self.copy_sources.shape
            or self.copy_positions.shape != (len(self.copy_sources), 2)
            or any(value.dtype != torch.int32
                   for value in (self.copy_sources, self.copy_destinations, self.copy_positions))
        ):
            raise ValueError("Context copies require aligned int32 metadata")
        binding = self.model_binding
        if binding is None:
            if model_runner is None:
                raise ValueError("Context prefill needs a native model binding")
            binding = getattr(model_runner, "context_model_binding", None)
            if binding is None:
                binding = ContextModelBinding(model_runner.model, model_runner.token_to_kv_pool,
                                              model_runner.kv_index_translator, page_size=1)
                model_runner.context_model_binding = binding
        return binding.bind(self)
