"""CPU model of the ZoomKV decode cache's token bookkeeping and selection
(oracle; TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Restates the default (``enable_offload=True``) path of
``S`` = Z/cache_hub/polar_cache_quest_density_single_layer_kivi.py on numpy
arrays:
  * lockstep prefill split into sink / retrieval / local (S:883-1006);
  * chunk metadata with the < chunk carry (S:2025-2157) using
    ``oracle.kivi.encode_chunks_ref`` per completed chunk;
  * live skipped tail and stage-1 sizes nk / n_dense (S:1798-1925);
  * flush of the oldest local tokens and window slide at layer 0 of the step
    after the near zone holds local + interval tokens (S:1379-1583);
  * compute: full attention below max(threshold, sink + local + 2 final_topk)
    tokens, else GQA mean -> Quest -> top-nk -> density -> top n_dense ->
    dense mask -> KIVI stage 2 -> global top-k + skipped (S:1589-1775,
    S:2195-2467, S:2688-2779), then attention over sink + local + selected
    tokens (float64 textbook attention);
  * kv_format "kivi4" (the 4-bit K + V retrieval zone, no reference
    counterpart): the same bookkeeping and selection; the attended retrieval
    rows are the exact dequant of each complete 32-token group's Format Q
    quantization, and bf16 for the last (retrieval length % 32) tokens.
"""
from __future__ import annotations

import math

import numpy as np

from . import select as osel
from .kivi import attention, dequant_kivi4, encode_chunks_ref, quantize_kivi4


class CacheModel:
    def __init__(self, layer_num, bs, kv, hq, input_length, max_new_length, sink, local, interval,
                 chunk, final_topk, full_threshold, cand_ratio, dense_ratio, dense_topk, sparse_topk,
                 max_skipped=512, force_cand_tokens=None, kv_format="bf16"):
        self.L, self.bs, self.kv, self.hq = layer_num, bs, kv, hq
        self.input_length, self.sink, self.local, self.interval = input_length, sink, local, interval
        self.chunk, self.final_topk, self.full_threshold = chunk, final_topk, full_threshold
        self.cand_ratio, self.dense_ratio = cand_ratio, dense_ratio
        self.dense_topk, self.sparse_topk = dense_topk, sparse_topk
        self.max_skipped, self.force_cand_tokens = max_skipped, force_cand_tokens
        assert kv_format in ("bf16", "kivi4")
        self.kv_format = kv_format
        cap = input_length + max_new_length
        near_cap = sink + local + interval
        self.near_cap = near_cap
        z = lambda n: [np.zeros((bs, kv, n, 128), np.float32) for _ in range(layer_num)]
        self.near_k, self.near_v = z(near_cap), z(near_cap)
        self.ret_k, self.ret_v = z(cap), z(cap)
        self.n_max = (cap + chunk - 1) // chunk
        self.mn, self.mx, self.mean = z(self.n_max), z(self.n_max), z(self.n_max)
        self.packed = [np.zeros((bs, kv, self.n_max, 16, chunk), np.int32) for _ in range(layer_num)]
        self.valid = [np.zeros((bs, kv, self.n_max), bool) for _ in range(layer_num)]
        self.carry_k = [np.zeros((bs, kv, chunk, 128), np.float32) for _ in range(layer_num)]
        self.carry = [0] * layer_num
        self.cpu_valid_end = [0] * layer_num
        self.seq = [0] * layer_num
        self.context = 0
        self.actual_retrieval = None
        self.nk = self.n_chunks = self.n_dense = 0
        self.skipped = np.zeros(0, np.int64)

    # -- stage-1 invariants (S:1798-1925) --
    def _cand_tokens(self, kv_len):
        c = self.chunk
        if kv_len <= 0:
            return 0
        if kv_len < c:
            return kv_len
        cap = (kv_len // c) * c
        target = self.force_cand_tokens if self.force_cand_tokens is not None else math.ceil(kv_len * self.cand_ratio)
        return min(cap, max(c, ((target + c - 1) // c) * c))

    def _refresh(self, kv_len):
        c = self.chunk
        covered = (kv_len // c) * c
        self.skipped = np.arange(covered, kv_len, dtype=np.int64)
        assert len(self.skipped) <= self.max_skipped
        if kv_len < c:
            self.n_chunks = self.nk = self.n_dense = 0
            return
        self.n_chunks = kv_len // c
        self.nk = max(1, min(self.n_chunks, self._cand_tokens(kv_len) // c))
        self.n_dense = max(1, int(self.nk * self.dense_ratio))

    # -- chunk metadata with carry (S:2025-2157) --
    def _encode(self, layer, block, chunk_start):
        n = block.shape[2] // self.chunk
        if n == 0:
            return
        mn, mx, mean, packed = encode_chunks_ref(block[:, :, :n * self.chunk], self.chunk)
        sl = slice(chunk_start, chunk_start + n)
        self.mn[layer][:, :, sl], self.mx[layer][:, :, sl], self.mean[layer][:, :, sl] = mn, mx, mean
        self.packed[layer][:, :, sl] = packed
        self.valid[layer][:, :, sl] = True

    def _store(self, layer, block, abs_start):
        c = self.chunk
        n = block.shape[2]
        if n <= 0:
            return
        carry = self.carry[layer]
        if carry:
            need = c - carry
            if n < need:
                self.carry_k[layer][:, :, carry:carry + n] = block
                self.carry[layer] = carry + n
                return
            merged = np.concatenate([self.carry_k[layer][:, :, :carry], block[:, :, :need]], axis=2)
            self._encode(layer, merged, (abs_start - carry) // c)
            block, abs_start, n = block[:, :, need:], abs_start + need, n - need
            self.carry[layer] = 0
            if n <= 0:
                return
        assert abs_start % c == 0
        usable = (n // c) * c
        self._encode(layer, block[:, :, :usable], abs_start // c)
        tail = n - usable
        self.carry_k[layer][:, :, :tail] = block[:, :, usable:]
        self.carry[layer] = tail

    # -- runtime entry points --
    def prefill(self, keys, values, layer, valid_start=0):
        """keys / values [bs, seq, kv, 128] (lockstep batch, S:883-1006)."""
        seq = keys.shape[1]
        k, v = np.swapaxes(keys, 1, 2), np.swapaxes(values, 1, 2)
        vs, s = valid_start, self.sink
        r0 = vs + s
        r1 = max(r0, seq - self.local)
        rlen = r1 - r0
        if self.actual_retrieval is None:
            self.actual_retrieval = rlen
            self._refresh(rlen)
        if rlen == 0:
            n = min(seq - vs, self.near_cap)
            self.near_k[layer][:, :, :n], self.near_v[layer][:, :, :n] = k[:, :, vs:vs + n], v[:, :, vs:vs + n]
            self.seq[layer] = n
        else:
            ll = seq - r1
            self.near_k[layer][:, :, :s], self.near_v[layer][:, :, :s] = k[:, :, vs:r0], v[:, :, vs:r0]
            self.near_k[layer][:, :, s:s + ll], self.near_v[layer][:, :, s:s + ll] = k[:, :, r1:seq], v[:, :, r1:seq]
            self.ret_k[layer][:, :, :rlen], self.ret_v[layer][:, :, :rlen] = k[:, :, r0:r1], v[:, :, r0:r1]
            self.cpu_valid_end[layer] = rlen
            self.seq[layer] = seq - vs
            self._store(layer, k[:, :, r0:r1], 0)
        if layer == self.L - 1:
            self.context += self.seq[layer]

    def _local_start(self):
        total = self.seq[0]
        steady = self.sink + self.local
        if self.input_length >= steady:
            buf = max(0, total - self.input_length) % self.interval
        elif total >= steady:
            buf = (total - steady) % self.interval
        else:
            buf = 0
        return max(self.sink, max(total - buf, self.sink) - self.local)

    def _flush(self):
        new_end = self._local_start()
        old_end = self.actual_retrieval + self.sink
        num = new_end - old_end
        assert num > 0
        self.actual_retrieval = new_end - self.sink
        self._refresh(self.actual_retrieval)
        s = self.sink
        for l in range(self.L):
            old_k = self.near_k[l][:, :, s:s + num].copy()
            old_v = self.near_v[l][:, :, s:s + num].copy()
            self._store(l, old_k, old_end - s)
            w0 = self.cpu_valid_end[l]
            self.ret_k[l][:, :, w0:w0 + num], self.ret_v[l][:, :, w0:w0 + num] = old_k, old_v
            self.cpu_valid_end[l] = w0 + num
            self.near_k[l][:, :, s:s + self.local] = self.near_k[l][:, :, s + num:s + self.local + num].copy()
            self.near_v[l][:, :, s:s + self.local] = self.near_v[l][:, :, s + num:s + self.local + num].copy()

    def decode_update(self, key, value, layer):
        """key / value [bs, 1, kv, 128] (S:1516-1583)."""
        cur = self.seq[layer]
        if layer == 0:
            near_len = cur - min(self.sink, cur) - self.cpu_valid_end[0]
            if near_len >= self.local + self.interval:
                self._flush()
        pos = cur - self.cpu_valid_end[layer]
        assert 0 <= pos < self.near_cap
        self.near_k[layer][:, :, pos], self.near_v[layer][:, :, pos] = key[:, 0], value[:, 0]
        self.seq[layer] = cur + 1
        if layer == self.L - 1:
            self.context += 1

    def select(self, raw_q, layer):
        """Retrieval-zone indices [bs, kv, min(final_topk, nk*chunk) + skipped]."""
        c = self.chunk
        sc = osel.quest_chunk_score(raw_q, self.mn[layer], self.mx[layer], self.n_chunks, self.valid[layer])
        cidx = np.clip(osel.topk_indices(sc, self.nk), 0, self.n_chunks - 1)
        dens = osel.chunk_density_scores(cidx, self.mean[layer], raw_q)
        dmask = osel.dense_mask_from_topk(osel.topk_indices(dens, self.n_dense), self.nk)
        vchunks = self.cpu_valid_end[layer] // c
        s2, i2 = osel.kivi_qk_dense_sparse(cidx, dmask, self.packed[layer][:, :, :vchunks], self.mn[layer],
                                           self.mx[layer], raw_q, max(1, min(self.dense_topk, c)),
                                           max(1, min(self.sparse_topk, c)), c)
        k = min(self.final_topk, s2.shape[-1])
        sk = np.broadcast_to(self.skipped, (self.bs, self.kv, len(self.skipped)))
        return osel.topk_gather_concat(s2, i2, sk, k, k + len(self.skipped))

    def retrieval_rows(self, layer):
        """The retrieval zone's K / V as attended [bs, kv, rlen, 128] (float64):
        bf16 rows, or with kv_format "kivi4" the complete 32-token groups as
        the exact dequant of their Format Q quantization (oracle.kivi) and
        the last rlen % 32 tokens as bf16 rows."""
        rlen = self.cpu_valid_end[layer]
        k = self.ret_k[layer][:, :, :rlen].astype(np.float64)
        v = self.ret_v[layer][:, :, :rlen].astype(np.float64)
        if self.kv_format == "kivi4":
            nq = rlen // 32 * 32
            if nq:
                kh, vh = dequant_kivi4(quantize_kivi4(self.ret_k[layer][:, :, :nq], self.ret_v[layer][:, :, :nq]))
                k[:, :, :nq], v[:, :, :nq] = kh, vh
        return k, v

    def compute(self, q, layer):
        """q [bs, 1, hq, 128] -> (out [bs, hq, 128] float64, selected indices or None)."""
        total = self.seq[layer]
        rlen = self.cpu_valid_end[layer]
        local_len = max(0, total - (self.sink + rlen))
        near_len = self.sink + local_len if rlen > 0 else min(total, self.near_cap)
        raw_q = osel.gqa_mean_query(q[:, 0], self.kv)
        min_total = max(self.full_threshold, self.sink + self.local + 2 * self.final_topk)
        full = total < min_total or rlen <= 0 or self.nk <= 0
        sel = None if full else self.select(raw_q, layer)
        out = np.zeros((self.bs, self.hq, 128))
        g = self.hq // self.kv
        ret_k, ret_v = self.retrieval_rows(layer)
        for b in range(self.bs):
            for h in range(self.kv):
                rows = np.arange(rlen) if full else sel[b, h]
                k = np.concatenate([ret_k[b, h, rows], self.near_k[layer][b, h, :near_len]])
                v = np.concatenate([ret_v[b, h, rows], self.near_v[layer][b, h, :near_len]])
                out[b, h * g:(h + 1) * g] = attention(q[b:b + 1, 0, h * g:(h + 1) * g], k[None, None], v[None, None],
                                                      1 / np.sqrt(128))[0]
        return out, sel
