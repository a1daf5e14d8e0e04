"""``polar_cache``: the ZoomKV decode cache as a drop-in for the reference's
``cache_hub.polar_cache_quest_density_single_layer_kivi.polar_cache`` (``S``).

The runtime picks the class by module name
(``importlib.import_module(cache_module).polar_cache``, ``Z/model_hub/qwen.py:336-350``),
so ``POLAR_CACHE_MODULE=zoomkv_revision_amd.cache`` (or ``"cache_module"`` in the
config) selects this implementation.  Constructor arguments, the methods the
runtime calls (``prefill_update_kv_cache``, ``sync``, ``decode_update_kv_cache``,
``compute``) and the ``context`` counter follow ``S:106-148, 863-877, 1516-1589,
2789-2793``.

Token bookkeeping is the reference's default ``enable_offload=True`` path:
  * a near zone ``[sink | local | update buffer]`` per layer and a retrieval
    zone ``[0, cpu_valid_end)`` of older tokens (global position sink + i);
  * prefill splits the prompt into sink / retrieval / local (``S:1009-1141``);
  * at the start of the decode step after the near zone holds
    ``local + interval`` tokens, the oldest ``interval`` local tokens are
    encoded, appended to the retrieval zone, and the local window slides
    (``S:1379-1512, 1516-1583``);
  * chunk min / max / centroid and 4-bit codes are written per completed
    chunk, with a carry of the < chunk tail (``S:2025-2157``), and the live
    tail is appended to every selection as "skipped" tokens (``S:1895-1925``).
Where the retrieval zone lives follows ``enable_offload`` (``S:519-611``):
  * ``enable_offload=True`` (the reference's default): in pinned host memory.
    A flush encodes the oldest local tokens on the device, stages them and
    moves them to their host rows on a copy stream, one pitched copy per K / V
    and layer, with a per-layer event (``S:1440-1474``); ``compute`` waits for
    that event on the device (no host synchronisation), gathers the selected
    rows over the host link into the first rows of the layer's device buffer
    (``h2d_gather_kv``) and attends them together with the near zone in one
    gather-attention launch (``S:1723-1750``).
  * ``enable_offload=False``: in device memory next to the near zone (a
    288 GB part holds it), so a flush is a device copy and ``compute`` attends
    the selected rows in place.
Both modes select the same tokens and give the same attention output (the
attended rows and their order are the same).

Per decode step and layer, ``compute`` runs (``S:1589-1775, 2195-2467, 2688-2779``):
GQA-mean query -> Quest chunk bounds -> top-nk chunks -> CDS density -> top
n_dense -> dense mask -> KIVI stage-2 scores -> fused global top-k + skipped
concat -> attention over sink + local + selected tokens; before
``max(full_attention_threshold, sink + local + 2 final_topk)`` tokens it
attends everything.
"""
from __future__ import annotations

import math
import os

import torch

from . import kivi
from .attention import gather_attention
from .gather import copy_rows, h2d_gather_kv, pinned_empty
from .quest import load_kernel_module as _load_quest
from .quest import QUEST_TOPK_MAX_CHUNKS, quest_chunk_score_gqa, quest_chunk_topk_gqa
from .rerank import partial_chunk_density_scores_cuda, topk_dense_mask
from .topk import float_topk_3d, float_topk_gather_concat_3d

_FALSY = ("0", "false", "False", "")


def _env_float_list(name: str, default: str):
    return [float(x.strip()) for x in os.environ.get(name, default).split(",") if x.strip()]


class polar_cache:
    """ZoomKV KIVI/Quest/CDS decode cache on gfx950 (see module docstring)."""

    def __init__(
        self,
        valid_start,
        layer_num: int,
        batch_size: int,
        max_length: int,
        num_key_value_heads: int,
        num_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        layer_mapping: dict,
        max_new_length: int,
        sink_size: int,
        local_size: int,
        core: int,
        nprobe: int,
        cache_unit_size: int,
        cache_cluster_num: int,
        num_gpus: int,
        model_size: int,
        codebook_path: str = "",
        collision_ratio: float = 0.3,
        candidate_ratio: float = 0.05,
        final_topk: int = 100,
        dynamic_update_interval: int = 512,
        full_attention_threshold: int = 2000,
        enable_offload: bool = True,
        debug_offload_coords: bool = False,
        enable_rerank: bool = False,
        enable_recall: bool = False,
        enable_alpha_correction: bool = False,
        enable_rerank_error_ablation: bool = False,
        enable_coarse_recall_ablation: bool = False,
        enable_rerank_recall_ablation: bool = False,
        adaptive_topk_enabled: bool = False,
        adaptive_topk_threshold: float = 0.9,
        adaptive_topk_min_k: int = 100,
        adaptive_topk_max_k: int = 400,
        kv_format: str | None = None,
    ) -> None:
        # knobs the reference accepts but this path does not use (S:125-148)
        del core, nprobe, cache_unit_size, cache_cluster_num, codebook_path, collision_ratio
        del debug_offload_coords, enable_rerank, enable_recall, enable_alpha_correction
        del enable_rerank_error_ablation, enable_coarse_recall_ablation, enable_rerank_recall_ablation
        del adaptive_topk_enabled, adaptive_topk_threshold, adaptive_topk_min_k, adaptive_topk_max_k
        if head_dim != 128:
            raise ValueError(f"head_dim must be 128 (got {head_dim})")
        if dtype != torch.bfloat16:
            raise ValueError(f"the KV cache dtype must be torch.bfloat16 (got {dtype})")
        # KV_Cache base attributes (Z/cache_hub/cache.py:9-45)
        self.layer_num = layer_num
        self.batch_size = batch_size
        self.max_length = max_length
        self.kv_head = num_key_value_heads
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.layer_mapping = layer_mapping
        self.num_gpus = num_gpus
        self.model_size = model_size
        self.context = 0
        # geometry (S:152-172)
        self.valid_start = valid_start
        self.sink_size = sink_size
        self.local_size = local_size
        self.steady_size = sink_size + local_size
        self.dynamic_update_interval = dynamic_update_interval if dynamic_update_interval is not None else local_size
        self.group_size = num_heads // num_key_value_heads
        self.max_new_length = max_new_length
        self.input_length = max_length - max_new_length
        self.FULL_ATTENTION_THRESHOLD = full_attention_threshold
        self.current_seq_len = [0] * layer_num
        self.candidate_ratio = candidate_ratio
        self.final_topk = final_topk
        self.enable_offload = bool(enable_offload)
        # storage of the retrieval zone (no reference counterpart: the
        # reference keeps bf16 K / V, S:561-571): "bf16", or "kivi4" for the
        # 4-bit K + V cache (Format Q, fp16 scale / zero) in HBM
        kv_format = kv_format if kv_format is not None else os.environ.get("POLAR_KV_FORMAT", "bf16")
        if kv_format not in ("bf16", "kivi4"):
            raise ValueError(f"kv_format must be 'bf16' or 'kivi4' (got {kv_format!r})")
        self.kv_format = kv_format
        self._kivi4 = kv_format == "kivi4"
        # Quest stage 1 / CDS knobs from the environment (S:178-292)
        self.quest_chunk_size = max(1, int(os.environ.get("POLAR_QUEST_CHUNK", "8")))
        if self.quest_chunk_size not in (8, 16):
            raise ValueError(f"POLAR_QUEST_CHUNK must be 8 or 16 (got {self.quest_chunk_size})")
        self.quest_coarse_candidate_ratio = float(os.environ.get("POLAR_QUEST_CAND_RATIO", "0.05"))
        self._dynamic_cand_enabled = os.environ.get("POLAR_QUEST_DYNAMIC_CAND_RATIO", "0") not in _FALSY
        self._dynamic_cand_thresholds, self._dynamic_cand_ratios = [], []
        if self._dynamic_cand_enabled:
            th = [int(x) for x in _env_float_list("POLAR_QUEST_DYNAMIC_CAND_THRESHOLDS", "5000,10000")]
            ra = _env_float_list("POLAR_QUEST_DYNAMIC_CAND_RATIOS", "0.7,0.5,0.4")
            if len(ra) != len(th) + 1:
                self._dynamic_cand_enabled = False   # the reference falls back to the fixed ratio
            else:
                self._dynamic_cand_thresholds, self._dynamic_cand_ratios = th, ra
        force = os.environ.get("POLAR_FORCE_CAND_TOKENS")
        self._force_cand_tokens = int(force) if force else None
        self.MAX_SKIPPED_INDICES = int(os.environ.get("POLAR_MAX_SKIPPED_INDICES", "512"))
        self.cds_dense_ratio = float(os.environ.get("POLAR_CDS_DENSE_RATIO", "0.1"))
        self.cds_dense_topk = int(os.environ.get("POLAR_CDS_DENSE_TOPK", "16"))
        self.cds_sparse_topk = int(os.environ.get("POLAR_CDS_SPARSE_TOPK", "8"))

        self.device = torch.device(list(layer_mapping.values())[0] if layer_mapping else "cuda:0")
        if self.device.type != "cuda":
            raise RuntimeError("polar_cache needs a GPU device")
        self._quest_kernel = _load_quest()   # fails loudly without the native library
        dev = dict(device=self.device)
        chunk = self.quest_chunk_size
        self.unified_kv_capacity = self.input_length + self.max_new_length
        # near zone [sink | local | update buffer]
        self.gpu_kv_capacity = sink_size + local_size + self.dynamic_update_interval
        self.cpu_kv_capacity = max(0, self.unified_kv_capacity - sink_size - local_size)
        bs, kv, d = batch_size, num_key_value_heads, head_dim
        self._min_total = max(self.FULL_ATTENTION_THRESHOLD, sink_size + local_size + self.final_topk * 2)
        if self._kivi4:
            # device rows: [retrieval tail | near zone].  The retrieval zone's
            # complete 32-token groups are Format Q records; its last
            # L % 32 tokens stay bf16, right-aligned in rows [0, 32), so that
            # they and the near zone are one run of rows.
            self._tail_rows = kivi.GROUP
            self._rows = self._tail_rows + self.gpu_kv_capacity
            self._near0 = self._tail_rows
            g_cap = max(1, (self.cpu_kv_capacity + kivi.GROUP - 1) // kivi.GROUP)
            self.kivi4_groups = [torch.zeros(bs, kv, g_cap, kivi.RECORD_WORDS, dtype=torch.int32, **dev)
                                 for _ in range(layer_num)]
            self.unified_keys_cpu = self.unified_values_cpu = None
            self._kivi4_stage = None                  # [tail | flushed tokens] staging, made on first use
        elif self.enable_offload:
            # device rows: [gathered retrieval rows | near zone]; the retrieval
            # zone in pinned host memory (S:519-611).  The gather area holds a
            # selection (final_topk + skipped) or, below the retrieval
            # threshold, the whole (short) retrieval zone.
            self._gather_rows = max(self.final_topk + self.MAX_SKIPPED_INDICES, self._min_total)
            self._rows = self._gather_rows + self.gpu_kv_capacity
            self._near0 = self._gather_rows
            cap = max(self.cpu_kv_capacity, 1)
            self.unified_keys_cpu = [pinned_empty((bs, kv, cap, d), dtype) for _ in range(layer_num)]
            self.unified_values_cpu = [pinned_empty((bs, kv, cap, d), dtype) for _ in range(layer_num)]
            self._copy_stream = torch.cuda.Stream(device=self.device)
            self._main_events = [torch.cuda.Event() for _ in range(layer_num)]
            self._copy_events = [torch.cuda.Event() for _ in range(layer_num)]
            for e in self._copy_events:           # recorded once: waiting on them is always valid
                e.record(torch.cuda.current_stream(self.device))
            n_buf = self.dynamic_update_interval
            self._offload_keys_buffer = [torch.empty(bs, kv, n_buf, d, dtype=dtype, **dev) for _ in range(layer_num)]
            self._offload_values_buffer = [torch.empty(bs, kv, n_buf, d, dtype=dtype, **dev)
                                           for _ in range(layer_num)]
        else:
            # device rows: [retrieval zone | near zone]
            self._rows = self.cpu_kv_capacity + self.gpu_kv_capacity
            self._near0 = self.cpu_kv_capacity
            self.unified_keys_cpu = self.unified_values_cpu = None
        self.unified_keys = [torch.zeros(bs, kv, self._rows, d, dtype=dtype, **dev) for _ in range(layer_num)]
        self.unified_values = [torch.zeros(bs, kv, self._rows, d, dtype=dtype, **dev) for _ in range(layer_num)]
        self.cpu_valid_end = [0] * layer_num      # retrieval-zone length per layer (name of S)
        self._arange_buffer = torch.arange(0, max(self.unified_kv_capacity, 1), dtype=torch.long, **dev)
        # chunk metadata (Format R) per layer (S:661-751)
        self._chunk_n_max = max(1, (self.unified_kv_capacity + chunk - 1) // chunk)
        n_max = self._chunk_n_max
        mk = lambda: torch.zeros(bs, kv, n_max, d, dtype=dtype, **dev)
        self._chunk_key_min_gpu = [mk() for _ in range(layer_num)]
        self._chunk_key_max_gpu = [mk() for _ in range(layer_num)]
        self._chunk_key_centroid_gpu = [mk() for _ in range(layer_num)]
        self._chunk_valid_mask_gpu = [torch.zeros(bs, kv, n_max, dtype=torch.bool, **dev) for _ in range(layer_num)]
        self.key_kivi_packed_gpu = [torch.zeros(bs, kv, n_max, 16, chunk, dtype=torch.int32, **dev)
                                    for _ in range(layer_num)]
        self._chunk_valid_end = [0] * layer_num
        self._chunk_carry_count = [0] * layer_num
        self._chunk_carry_keys = [torch.zeros(bs, kv, max(chunk - 1, 1), d, dtype=dtype, **dev)
                                  for _ in range(layer_num)]
        self._chunk_merge_buffer = [torch.empty(bs, kv, chunk, d, dtype=dtype, **dev) for _ in range(layer_num)]
        self._chunk_skipped_indices_gpu = [torch.zeros(bs, kv, self.MAX_SKIPPED_INDICES, dtype=torch.int64, **dev)
                                           for _ in range(layer_num)]
        self._chunk_skipped_count = [0] * layer_num
        self._quest_scores_buffer = torch.empty(bs * kv * n_max, dtype=torch.float32, **dev)
        self._actual_retrieval_length = None
        self._cached_quest_nk = 0
        self._cached_quest_n_chunks = 0
        self._cached_region_total_len = -1
        self._cached_region_info = None
        self._decode_step_counter = 0
        self._raw_q = torch.empty(bs, kv, d, dtype=dtype, **dev)
        self._last_topk_indices = None

    # ------------------------------------------------------------------
    # prefill (S:863-1141)
    # ------------------------------------------------------------------
    def prefill_update_kv_cache(self, query_states, key_states, value_states, layer_idx, batch_idx):
        """key_states / value_states [bsz, seq_len, kv, 128]; bsz == 1 writes
        batch row batch_idx, bsz == batch_size writes all rows (on batch_idx 0).
        Returns the inputs without their left padding (S:863-877)."""
        del query_states
        bsz = key_states.shape[0]
        if bsz == 1:
            vs = int(self.valid_start[batch_idx]) if hasattr(self.valid_start, "__len__") else int(self.valid_start)
            rows = slice(batch_idx, batch_idx + 1)
            last = batch_idx + bsz == self.batch_size
        else:
            vs = int(self.valid_start[0]) if hasattr(self.valid_start, "__len__") else int(self.valid_start)
            if batch_idx != 0:
                return key_states[:, vs:], value_states[:, vs:]
            if bsz != self.batch_size:
                raise ValueError(f"bsz ({bsz}) must equal cache batch_size ({self.batch_size})")
            if hasattr(self.valid_start, "__len__"):
                if any(int(self.valid_start[b]) != vs for b in range(bsz)):
                    raise ValueError("lockstep multi-batch prefill needs the same valid_start across the batch")
            rows = slice(0, bsz)
            last = True
        self._prefill(key_states, value_states, layer_idx, rows, vs)
        if layer_idx == self.layer_num - 1 and last:
            self.context += self.current_seq_len[layer_idx]
        return key_states[:, vs:], value_states[:, vs:]

    def _prefill(self, key_states, value_states, layer_idx, rows, vs):
        seq_len = key_states.shape[1]
        if seq_len > self.input_length:
            raise ValueError(f"prefill of {seq_len} tokens exceeds input_length {self.input_length}")
        sink_end = vs + self.sink_size
        retrieval_start = sink_end
        retrieval_end = max(retrieval_start, seq_len - self.local_size)
        retrieval_length = retrieval_end - retrieval_start
        if self._actual_retrieval_length is None:
            self._actual_retrieval_length = retrieval_length
            self._refresh_quest_chunk_cache(retrieval_length)
        K, V = self.unified_keys[layer_idx], self.unified_values[layer_idx]
        kt, vt = key_states.transpose(1, 2), value_states.transpose(1, 2)     # [bsz, kv, seq, d]
        n0 = self._near0
        if retrieval_length == 0:                                          # short prompt: all near zone
            n = min(seq_len - vs, self.gpu_kv_capacity)
            K[rows, :, n0:n0 + n] = kt[:, :, vs:vs + n].to(self.dtype)
            V[rows, :, n0:n0 + n] = vt[:, :, vs:vs + n].to(self.dtype)
            self.current_seq_len[layer_idx] = n
            return
        local_len = seq_len - retrieval_end
        K[rows, :, n0:n0 + self.sink_size] = kt[:, :, vs:sink_end].to(self.dtype)
        V[rows, :, n0:n0 + self.sink_size] = vt[:, :, vs:sink_end].to(self.dtype)
        K[rows, :, n0 + self.sink_size:n0 + self.sink_size + local_len] = kt[:, :, retrieval_end:seq_len].to(self.dtype)
        V[rows, :, n0 + self.sink_size:n0 + self.sink_size + local_len] = vt[:, :, retrieval_end:seq_len].to(self.dtype)
        kr = kt[:, :, retrieval_start:retrieval_end].to(self.dtype)
        vr = vt[:, :, retrieval_start:retrieval_end].to(self.dtype)
        if self._kivi4:
            # complete groups to Format Q, the < 32-token rest to the tail rows
            ng = kivi.kivi4_pack(kr, vr, self._kivi4_view(layer_idx, rows), 0)
            t = retrieval_length - kivi.GROUP * ng
            T = self._tail_rows
            if t:
                K[rows, :, T - t:T] = kr[:, :, kivi.GROUP * ng:]
                V[rows, :, T - t:T] = vr[:, :, kivi.GROUP * ng:]
        elif self.enable_offload:
            # the prompt's retrieval zone to its pinned host rows (S:1003-1141)
            torch.cuda.current_stream(self.device).wait_event(self._copy_events[layer_idx])
            self.unified_keys_cpu[layer_idx][rows, :, :retrieval_length].copy_(kr)
            self.unified_values_cpu[layer_idx][rows, :, :retrieval_length].copy_(vr)
        else:
            K[rows, :, :retrieval_length] = kr
            V[rows, :, :retrieval_length] = vr
        self.cpu_valid_end[layer_idx] = retrieval_length
        self.current_seq_len[layer_idx] = seq_len - vs
        # a prefill writes its rows' retrieval zone from offset 0: no earlier
        # carry belongs to them (the reference's per-layer carry would leak the
        # previous row's tail into a one-row prefill)
        self._chunk_carry_count[layer_idx] = 0
        self._store_chunks(layer_idx, kr, 0, rows)

    def sync(self, layer_idx, batch_idx):
        """Nothing to wait for: every write is on the caller's stream (S:2789-2793)."""
        del layer_idx, batch_idx

    # ------------------------------------------------------------------
    # chunk metadata with carry (S:2025-2157)
    # ------------------------------------------------------------------
    def _encode(self, layer_idx, keys, chunk_start, rows):
        n = kivi.chunk_encode(keys, self.quest_chunk_size, chunk_start,
                              self._chunk_key_min_gpu[layer_idx][rows], self._chunk_key_max_gpu[layer_idx][rows],
                              self._chunk_key_centroid_gpu[layer_idx][rows],
                              self._chunk_valid_mask_gpu[layer_idx][rows], self.key_kivi_packed_gpu[layer_idx][rows])
        self._chunk_valid_end[layer_idx] = max(self._chunk_valid_end[layer_idx], chunk_start + n)

    def _store_chunks(self, layer_idx, key_block, abs_token_start, rows):
        """Encode the completed chunks of key_block ([bs_rows, kv, n, 128], at
        retrieval-zone offset abs_token_start), merging the carried tail first
        and carrying the new < chunk tail."""
        chunk = self.quest_chunk_size
        n = key_block.shape[2]
        if n <= 0:
            return
        carry = self._chunk_carry_count[layer_idx]
        if carry > 0:
            need = chunk - carry
            ck = self._chunk_carry_keys[layer_idx]
            if n < need:
                ck[rows, :, carry:carry + n].copy_(key_block)
                self._chunk_carry_count[layer_idx] = carry + n
                return
            merge = self._chunk_merge_buffer[layer_idx][rows]
            merge[:, :, :carry].copy_(ck[rows, :, :carry])
            merge[:, :, carry:].copy_(key_block[:, :, :need])
            self._check_chunk_capacity(layer_idx, (abs_token_start - carry) // chunk + 1)
            self._encode(layer_idx, merge, (abs_token_start - carry) // chunk, rows)
            key_block = key_block[:, :, need:]
            abs_token_start += need
            n -= need
            self._chunk_carry_count[layer_idx] = 0
            if n <= 0:
                return
        if abs_token_start % chunk:
            raise RuntimeError(f"misaligned chunk start {abs_token_start} without carry (layer {layer_idx})")
        usable = (n // chunk) * chunk
        if usable:
            self._check_chunk_capacity(layer_idx, abs_token_start // chunk + usable // chunk)
            self._encode(layer_idx, key_block[:, :, :usable], abs_token_start // chunk, rows)
        tail = n - usable
        if tail:
            self._chunk_carry_keys[layer_idx][rows, :, :tail].copy_(key_block[:, :, usable:])
        self._chunk_carry_count[layer_idx] = tail

    def _check_chunk_capacity(self, layer_idx, chunk_end):
        if chunk_end > self._chunk_n_max:
            raise RuntimeError(f"layer {layer_idx}: chunk {chunk_end} exceeds capacity {self._chunk_n_max}")

    # ------------------------------------------------------------------
    # stage-1 invariants (S:1798-1925)
    # ------------------------------------------------------------------
    def _quest_candidate_ratio(self, kv_len: int) -> float:
        if not self._dynamic_cand_enabled:
            return self.quest_coarse_candidate_ratio
        for threshold, ratio in zip(self._dynamic_cand_thresholds, self._dynamic_cand_ratios):
            if kv_len < threshold:
                return ratio
        return self._dynamic_cand_ratios[-1]

    def _quest_aligned_candidate_tokens(self, kv_len: int) -> int:
        c = self.quest_chunk_size
        if kv_len <= 0:
            return 0
        if kv_len < c:
            return kv_len
        cap = (kv_len // c) * c
        target = self._force_cand_tokens if self._force_cand_tokens is not None else \
            math.ceil(kv_len * self._quest_candidate_ratio(kv_len))
        return min(cap, max(c, ((target + c - 1) // c) * c))

    def _refresh_quest_chunk_cache(self, kv_len: int):
        chunk = self.quest_chunk_size
        self._refresh_live_skipped_indices(kv_len)
        if kv_len < chunk:
            self._cached_quest_n_chunks = 0
            self._cached_quest_nk = 0
            self._cached_cds_n_dense = 0
            return
        n_chunks = kv_len // chunk
        nk = max(1, min(n_chunks, self._quest_aligned_candidate_tokens(kv_len) // chunk))
        self._cached_quest_n_chunks = n_chunks
        self._cached_quest_nk = nk
        bs, kv, dev = self.batch_size, self.kv_head, self.device
        self._cached_scores_view = self._quest_scores_buffer[:bs * kv * n_chunks].view(bs, kv, n_chunks)
        self._cached_cds_n_dense = max(1, int(nk * self.cds_dense_ratio))
        self._cached_chunk_idx = torch.empty(bs, kv, nk, dtype=torch.int64, device=dev)
        self._cached_dense_mask = torch.zeros(bs, kv, nk, dtype=torch.bool, device=dev)
        self._cached_cds_out_scores = torch.empty(bs, kv, nk * chunk, dtype=torch.float32, device=dev)
        self._cached_cds_out_indices = torch.empty(bs, kv, nk * chunk, dtype=torch.int64, device=dev)
        self._cached_cds_density_scores = torch.empty(bs, kv, nk, dtype=torch.float32, device=dev)
        self._cached_cds_final_indices = torch.empty(bs, kv, self.final_topk + self.MAX_SKIPPED_INDICES,
                                                     dtype=torch.int64, device=dev)

    def _refresh_live_skipped_indices(self, kv_len: int):
        kv_len = max(0, int(kv_len))
        chunk = self.quest_chunk_size
        covered = (kv_len // chunk) * chunk
        sk = kv_len - covered
        if sk > self.MAX_SKIPPED_INDICES:
            raise RuntimeError(f"live skipped indices overflow: {sk} > {self.MAX_SKIPPED_INDICES}")
        row = torch.arange(covered, kv_len, device=self.device, dtype=torch.int64) if sk else None
        for ldx in range(self.layer_num):
            self._chunk_skipped_count[ldx] = sk
            if row is not None:
                self._chunk_skipped_indices_gpu[ldx][:, :, :sk].copy_(row)

    # ------------------------------------------------------------------
    # regions (S:1173-1277)
    # ------------------------------------------------------------------
    def get_region_indices(self, layer_idx, device=None):
        del device
        total = self.current_seq_len[layer_idx]
        if total == self._cached_region_total_len and self._cached_region_info is not None:
            return self._cached_region_info
        retrieval_length = int(self.cpu_valid_end[layer_idx])
        local_start = self.sink_size + retrieval_length
        local_len = max(0, total - local_start)
        info = {
            "sink_indices": self._arange_buffer[:self.sink_size],
            "local_indices": self._arange_buffer[local_start:total] if local_len > 0 else self._arange_buffer[:0],
            "retrieval_start": self.sink_size,
            "retrieval_length": retrieval_length,
            "total_len": total,
            "local_len": local_len,
        }
        self._cached_region_total_len = total
        self._cached_region_info = info
        return info

    def _compute_local_start(self, layer_idx=0):
        total = self.current_seq_len[layer_idx]
        if self.input_length >= self.steady_size:
            buf = max(0, total - self.input_length) % self.dynamic_update_interval
        elif total >= self.steady_size:
            buf = (total - self.steady_size) % self.dynamic_update_interval
        else:
            buf = 0
        local_end = max(total - buf, self.sink_size)
        return max(self.sink_size, local_end - self.local_size)

    # ------------------------------------------------------------------
    # flush (S:1379-1512) and decode append (S:1516-1583)
    # ------------------------------------------------------------------
    def _update_polar_index(self):
        new_end = self._compute_local_start(0)
        old_end = self._actual_retrieval_length + self.sink_size
        num_new = new_end - old_end
        if num_new <= 0:
            raise RuntimeError(f"flush of {num_new} tokens: inconsistent cache state")
        self._actual_retrieval_length = new_end - self.sink_size
        self._refresh_quest_chunk_cache(self._actual_retrieval_length)
        s, n0, loc = self.sink_size, self._near0, self.local_size
        for ldx in range(self.layer_num):
            K, V = self.unified_keys[ldx], self.unified_values[ldx]
            oldest = slice(n0 + s, n0 + s + num_new)
            self._store_chunks(ldx, K[:, :, oldest], old_end - s, slice(0, self.batch_size))
            w0 = self.cpu_valid_end[ldx]
            if w0 + num_new > self.cpu_kv_capacity:
                raise RuntimeError(f"layer {ldx}: retrieval zone full ({w0} + {num_new} > {self.cpu_kv_capacity})")
            if self._kivi4:
                self._flush_kivi4(ldx, K[:, :, oldest], V[:, :, oldest], w0, num_new)
            elif self.enable_offload:
                self._offload(ldx, K[:, :, oldest], V[:, :, oldest], w0, num_new)
            else:
                K[:, :, w0:w0 + num_new].copy_(K[:, :, oldest])
                V[:, :, w0:w0 + num_new].copy_(V[:, :, oldest])
            self.cpu_valid_end[ldx] = w0 + num_new
            # slide: [sink + num_new, sink + local + num_new) -> [sink, sink + local)
            src = slice(n0 + s + num_new, n0 + s + loc + num_new)
            dst = slice(n0 + s, n0 + s + loc)
            K[:, :, dst] = K[:, :, src].clone()
            V[:, :, dst] = V[:, :, src].clone()
        self._cached_region_total_len = -1
        self._cached_region_info = None

    def _kivi4_view(self, ldx, rows=slice(None)):
        """The layer's Format Q records as a Kivi4Cache (for the pack)."""
        return kivi.Kivi4Cache(self.kivi4_groups[ldx][rows], self.unified_keys[ldx][rows],
                               self.unified_values[ldx][rows])

    def _flush_kivi4(self, ldx, k_old, v_old, w0, n):
        """Append n flushed tokens to the 4-bit retrieval zone [0, w0): the
        bf16 tail of w0 % 32 tokens and the new tokens are packed into
        complete groups from group w0 // 32 on, and the rest becomes the new
        tail (rows [32 - t, 32))."""
        G, T = kivi.GROUP, self._tail_rows
        t = w0 % G
        K, V = self.unified_keys[ldx], self.unified_values[ldx]
        if t:
            bs, kv, _, d = K.shape
            if self._kivi4_stage is None or self._kivi4_stage[0].shape[2] < t + n:
                self._kivi4_stage = [torch.empty(bs, kv, t + n, d, dtype=self.dtype, device=self.device)
                                     for _ in range(2)]
            sk, sv = self._kivi4_stage[0][:, :, :t + n], self._kivi4_stage[1][:, :, :t + n]
            sk[:, :, :t].copy_(K[:, :, T - t:T])
            sv[:, :, :t].copy_(V[:, :, T - t:T])
            sk[:, :, t:].copy_(k_old)
            sv[:, :, t:].copy_(v_old)
        else:
            sk, sv = k_old, v_old
        ng = kivi.kivi4_pack(sk, sv, self._kivi4_view(ldx), w0 // G)
        t2 = t + n - G * ng
        if t2:
            K[:, :, T - t2:T].copy_(sk[:, :, G * ng:])
            V[:, :, T - t2:T].copy_(sv[:, :, G * ng:])

    def check_range(self) -> None:
        """kivi4 storage: raise RuntimeError if any pack since the last check
        met values beyond the 4-bit cache's fp16 range (kivi.kivi4_pack); reads
        a device word, so it waits for the queued work (call it where the
        caller synchronises anyway)."""
        if self._kivi4:
            kivi.check_kivi4_pack_range(self.device)

    def _offload(self, ldx, k_old, v_old, w0, n):
        """Stage the n oldest near-zone tokens and move them to host rows
        [w0, w0 + n) on the copy stream (S:1440-1474); _copy_events[ldx] marks
        the end of the move."""
        main = torch.cuda.current_stream(self.device)
        main.wait_event(self._copy_events[ldx])         # the staging buffer's previous move is done
        sk = self._offload_keys_buffer[ldx][:, :, :n]
        sv = self._offload_values_buffer[ldx][:, :, :n]
        sk.copy_(k_old)
        sv.copy_(v_old)
        self._main_events[ldx].record(main)
        self._copy_stream.wait_event(self._main_events[ldx])
        with torch.cuda.stream(self._copy_stream):
            copy_rows(self.unified_keys_cpu[ldx][:, :, w0:w0 + n], sk)
            copy_rows(self.unified_values_cpu[ldx][:, :, w0:w0 + n], sv)
            self._copy_events[ldx].record(self._copy_stream)

    def decode_update_kv_cache(self, key_states, value_states, layer_idx):
        """Append one token ([bs, 1, kv, 128]) of one layer; the flush runs at
        layer 0 of the step after the near zone filled.  Returns (None, None)."""
        row = self.decode_reserve_row(layer_idx)
        self.unified_keys[layer_idx][:, :, row] = key_states[:, 0].to(self.dtype)
        self.unified_values[layer_idx][:, :, row] = value_states[:, 0].to(self.dtype)
        return None, None

    def decode_reserve_row(self, layer_idx) -> int:
        """The bookkeeping of decode_update_kv_cache without the write: runs the
        flush when due, commits the token and returns the row of
        unified_keys[layer_idx] / unified_values[layer_idx] ([bs, kv, rows,
        128]) that the token's K / V must be written to (before the next
        compute of this layer)."""
        cur = self.current_seq_len[layer_idx]
        if layer_idx == 0:
            near_len = cur - min(self.sink_size, cur) - int(self.cpu_valid_end[0])
            if near_len >= self.local_size + self.dynamic_update_interval:
                if not all(n == cur for n in self.current_seq_len):
                    raise RuntimeError(f"cache flush requires all layer lengths to match: {self.current_seq_len}")
                self._update_polar_index()
        pos = cur - int(self.cpu_valid_end[layer_idx])
        if not 0 <= pos < self.gpu_kv_capacity:
            raise RuntimeError(f"near-zone write at {pos} outside [0, {self.gpu_kv_capacity}) (layer {layer_idx})")
        self.current_seq_len[layer_idx] = cur + 1
        if layer_idx == self.layer_num - 1:
            if not all(n == self.current_seq_len[0] for n in self.current_seq_len):
                raise RuntimeError(f"decode step layer lengths diverged: {self.current_seq_len}")
            self._decode_step_counter += 1
            self.context += 1
        return self._near0 + pos

    # ------------------------------------------------------------------
    # decode attention (S:1589-1775) and selection (S:2195-2467, 2688-2779)
    # ------------------------------------------------------------------
    def _stage2_out_width(self, layer_idx) -> int | None:
        """Lanes per chunk that stage 2 writes (its compact output), or None
        for the full chunk.  Only the kept lanes are written when the global
        top-k cannot reach a (-1e30, 0) filler: every chunk id is in range
        (the packed chunks cover the Quest chunks) and the chunks keep at least
        final_topk tokens.  The top-k then reads half the entries at the
        production knobs (8 of 16) and picks the same tokens."""
        chunk = self.quest_chunk_size
        n_chunks, nk = self._cached_quest_n_chunks, self._cached_quest_nk
        dense_topk = max(1, min(self.cds_dense_topk, chunk))
        sparse_topk = max(1, min(self.cds_sparse_topk, chunk))
        width = max(dense_topk, sparse_topk)
        valid_chunks = int(self.cpu_valid_end[layer_idx]) // chunk
        if width < chunk and valid_chunks >= n_chunks and nk * min(dense_topk, sparse_topk) >= self.final_topk:
            return width
        return None

    def _select(self, queries, layer_idx):
        """GQA-mean query + Quest stage 1 (one launch) + CDS dense / sparse +
        KIVI stage 2 + global top-k: retrieval-zone token indices
        [bs, kv, min(final_topk, nk*chunk) + skipped]."""
        bs, chunk = self.batch_size, self.quest_chunk_size
        n_chunks, nk = self._cached_quest_n_chunks, self._cached_quest_nk
        scores = self._cached_scores_view
        # raw_q = mean over each KV head's query heads (S:1621-1626), formed by
        # the Quest scan (S:2223) itself
        # the reference clamps to [0, n_chunks); with nk <= n_chunks every
        # index of the top-k is already inside, so the clamp (a launch) is skipped
        if n_chunks <= QUEST_TOPK_MAX_CHUNKS:
            # GQA mean + bounds + top-nk chunks in one launch
            raw_q = self._raw_q
            chunk_idx = quest_chunk_topk_gqa(queries, self.kv_head, self._chunk_key_min_gpu[layer_idx],
                                             self._chunk_key_max_gpu[layer_idx], scores, n_chunks,
                                             self._chunk_valid_mask_gpu[layer_idx], raw_q, nk,
                                             self._cached_chunk_idx)
        else:
            raw_q = quest_chunk_score_gqa(queries, self.kv_head, self._chunk_key_min_gpu[layer_idx],
                                          self._chunk_key_max_gpu[layer_idx], scores, n_chunks,
                                          self._chunk_valid_mask_gpu[layer_idx], self._raw_q)
            chunk_idx = float_topk_3d(scores, nk)
        dense_topk = max(1, min(self.cds_dense_topk, chunk))
        sparse_topk = max(1, min(self.cds_sparse_topk, chunk))
        dense_mask = self._cached_dense_mask
        if dense_topk != sparse_topk:
            density = self._cached_cds_density_scores
            partial_chunk_density_scores_cuda(chunk_idx, self._chunk_key_centroid_gpu[layer_idx], raw_q, density)
            # float_topk_3d + dense_mask_from_topk_cuda (S:2360-2369) in one launch
            topk_dense_mask(density, self._cached_cds_n_dense, dense_mask)
        # else: every chunk keeps the same number of tokens whichever class it
        # is in, so the density classification (S:2352-2369) cannot change the
        # stage-2 output and its two launches are skipped
        valid_chunks = int(self.cpu_valid_end[layer_idx]) // chunk
        packed = self.key_kivi_packed_gpu[layer_idx][:, :, :valid_chunks]
        out_scores, out_indices = self._cached_cds_out_scores, self._cached_cds_out_indices
        width = self._stage2_out_width(layer_idx)
        if width is not None:
            out_scores, out_indices = out_scores[:, :, :nk * width], out_indices[:, :, :nk * width]
        kivi.partial_chunk_kivi_qk_dense_sparse_cuda(
            chunk_idx, dense_mask, packed, self._chunk_key_min_gpu[layer_idx], self._chunk_key_max_gpu[layer_idx],
            raw_q, dense_topk, sparse_topk, chunk, out_scores, out_indices, out_width=width)
        k = min(self.final_topk, out_scores.shape[-1])
        sk = self._chunk_skipped_count[layer_idx]
        skipped = self._chunk_skipped_indices_gpu[layer_idx][:bs, :, :sk]
        out = self._cached_cds_final_indices[:bs]
        float_topk_gather_concat_3d(out_scores, out_indices, skipped, out, k)
        return out[:, :, :k + sk]

    def compute(self, queries, layer_idx):
        """queries [bs, 1, num_heads, 128] bf16 -> attention output of the same shape."""
        region = self.get_region_indices(layer_idx)
        total = region["total_len"]
        local_len = region["local_len"]
        retrieval_len = int(self.cpu_valid_end[layer_idx])
        K, V = self.unified_keys[layer_idx], self.unified_values[layer_idx]
        bs = self.batch_size
        if retrieval_len > 0:
            near_len = self.sink_size + local_len
        else:
            near_len = min(total, self.gpu_kv_capacity)      # short prompt: everything sits in the near zone
        full = total < self._min_total or retrieval_len <= 0 or self._cached_quest_nk <= 0
        if self._kivi4:
            return self._compute_kivi4(queries, layer_idx, retrieval_len, near_len, full)
        if full:
            idx = self._arange_buffer[:retrieval_len].view(1, 1, -1).expand(bs, self.kv_head, -1)
            self._last_topk_indices = None
        else:
            idx = self._select(queries, layer_idx)
            self._last_topk_indices = idx
        n = idx.shape[-1]
        if self.enable_offload and n:
            # the listed host rows into device rows [0, n) (S:1723-1733), after
            # this layer's last move to the host
            torch.cuda.current_stream(self.device).wait_event(self._copy_events[layer_idx])
            h2d_gather_kv(self.unified_keys_cpu[layer_idx], self.unified_values_cpu[layer_idx], idx, K, V)
            idx = self._arange_buffer[:n].view(1, 1, -1).expand(bs, self.kv_head, -1)
        return gather_attention(queries, K, V, idx if n else None, self._near0, near_len)

    def _compute_kivi4(self, queries, layer_idx, retrieval_len, near_len, full):
        """compute with the 4-bit retrieval zone: the same selection, then one
        launch over the selected tokens (Format Q groups, or the bf16 tail) and
        the near zone; below the retrieval threshold, the dense 4-bit kernel
        over every group plus the tail and near rows (one run of rows)."""
        G, T = kivi.GROUP, self._tail_rows
        ng, t = retrieval_len // G, retrieval_len % G
        K, V = self.unified_keys[layer_idx], self.unified_values[layer_idx]
        if full:
            self._last_topk_indices = None
            view = kivi.Kivi4Cache(self.kivi4_groups[layer_idx], K[:, :, T - t:], V[:, :, T - t:])
            return kivi.kivi4_decode_attention(queries, view, ng, t + near_len)
        idx = self._select(queries, layer_idx)
        self._last_topk_indices = idx
        return kivi.kivi4_token_attention(queries, self.kivi4_groups[layer_idx], ng, K, V, idx, T - t, t, T,
                                          near_len)
