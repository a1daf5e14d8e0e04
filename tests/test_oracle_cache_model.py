"""Pins of the CPU cache model (oracle/cache_model.py) by closed forms of the
reference's bookkeeping (S = Z/cache_hub/polar_cache_quest_density_single_layer_kivi.py):

* flush schedule (S:1262-1277 _compute_local_start, S:1532-1544 the layer-0
  trigger near_len >= local + interval, S:1379-1400 num_new_tokens): with the
  prompt filling input_length, a flush runs before the write of decode step
  n = k * interval (k >= 1) and leaves cpu_valid_end = R0 + k * interval,
  R0 = max(0, prompt - sink - local); with a prompt shorter than sink + local
  it runs when the sequence first holds sink + local + k * interval tokens
  and leaves cpu_valid_end = k * interval;
* token placement: the retrieval zone row i holds token sink + i and the near
  zone holds the sink then tokens [sink + cpu_valid_end, total) in order
  (every token exactly once);
* chunk metadata: chunk j = tokens [sink + j*c, sink + (j+1)*c) of the
  sequence, whatever the carry did, and only chunks below
  floor(cpu_valid_end / c) are valid; the skipped tail is the rest
  (S:1895-1925);
* stage-1 sizes: nk = min(n_chunks, align_c(max(c, ceil(L * ratio))) / c)
  and n_dense = max(1, int(nk * dense_ratio)) (S:1798-1825, S:1866-1870).

Keys carry their own token position in channel 0 (exactly representable in
bf16 below 256; channel 1 holds the position / 256), so every check is an
exact comparison with the input sequence.
"""
import math

import numpy as np
import pytest

from oracle.cache_model import CacheModel
from oracle.kivi import encode_chunks_ref


def _tok_keys(pos: np.ndarray, bs: int, kv: int) -> np.ndarray:
    """[bs, n, kv, 128] keys whose channels 0 / 1 encode the token position."""
    n = pos.shape[0]
    k = np.zeros((bs, n, kv, 128), np.float32)
    k[:, :, :, 0] = (pos % 256)[None, :, None]
    k[:, :, :, 1] = (pos // 256)[None, :, None]
    k[:, :, :, 2:] = ((pos[None, :, None, None] * 7 + np.arange(126)) % 13 - 6).astype(np.float32)
    return k


def _decode_pos(rows: np.ndarray) -> np.ndarray:
    return (rows[..., 0] + 256 * rows[..., 1]).astype(np.int64)


def _drive(prompt, inp, new, sink, local, interval, chunk, steps, L=2):
    bs, kv, hq = 1, 1, 4
    m = CacheModel(L, bs, kv, hq, inp, new, sink, local, interval, chunk, final_topk=8,
                   full_threshold=10 ** 9, cand_ratio=0.25, dense_ratio=0.3, dense_topk=chunk,
                   sparse_topk=chunk)
    k = _tok_keys(np.arange(prompt), bs, kv)
    for l in range(L):
        m.prefill(k, k, l)
    flushes = []
    for n in range(steps):
        before = m.cpu_valid_end[0]
        kt = _tok_keys(np.array([prompt + n]), bs, kv)
        for l in range(L):
            m.decode_update(kt, kt, l)
        if m.cpu_valid_end[0] != before:
            flushes.append((n, m.cpu_valid_end[0]))
        _check_placement(m, prompt + n + 1, sink, chunk, L)
    return m, flushes


def _check_placement(m, total, sink, chunk, L):
    for l in range(L):
        assert m.seq[l] == total
        r = m.cpu_valid_end[l]
        assert np.array_equal(_decode_pos(m.ret_k[l][0, 0, :r]), sink + np.arange(r))
        if r > 0:
            near = _decode_pos(m.near_k[l][0, 0, :total - r])
            assert np.array_equal(near, np.r_[np.arange(sink), np.arange(sink + r, total)])
        nc = r // chunk
        assert m.valid[l][0, 0, :nc].all() and not m.valid[l][0, 0, nc:].any()
        if nc:
            ret = m.ret_k[l][:, :, :nc * chunk]
            mn, mx, mean, packed = encode_chunks_ref(ret, chunk)
            assert np.array_equal(m.mn[l][:, :, :nc], mn) and np.array_equal(m.mx[l][:, :, :nc], mx)
            # with the placement check above: chunk j is tokens sink + j*c .. sink + j*c + c - 1
            assert np.array_equal(m.packed[l][:, :, :nc], packed)
        assert np.array_equal(m.skipped, np.arange(nc * chunk, m.actual_retrieval))


@pytest.mark.parametrize("sink,local,interval,chunk", [(4, 16, 8, 8), (4, 16, 12, 8), (6, 20, 10, 16)])
def test_flush_schedule_long_prompt(sink, local, interval, chunk):
    prompt = 90                              # >= sink + local; fills input_length
    _, flushes = _drive(prompt, prompt, 80, sink, local, interval, chunk, steps=5 * interval + 3)
    r0 = prompt - sink - local
    want = [(k * interval, r0 + k * interval) for k in range(1, 6)]
    assert flushes == want


@pytest.mark.parametrize("sink,local,interval,chunk", [(4, 16, 8, 8), (4, 16, 12, 8)])
def test_flush_schedule_short_prompt(sink, local, interval, chunk):
    prompt = 11                              # < sink + local: everything starts in the near zone
    _, flushes = _drive(prompt, prompt, 90, sink, local, interval, chunk, steps=4 * interval + sink + local)
    want = [(sink + local + k * interval - prompt, k * interval) for k in range(1, 5)]
    assert flushes[:4] == want


def test_stage1_sizes_closed_form():
    for c in (8, 16):
        for ratio in (0.05, 0.25, 0.4, 0.7):
            m = CacheModel(1, 1, 1, 4, 64, 8, 4, 16, 8, c, 8, 10 ** 9, ratio, 0.3, c, c)
            for L in (0, 3, c - 1, c, c + 1, 5 * c + 3, 37, 1000, 4097, 65472):
                m._refresh(L)
                if L < c:
                    assert (m.n_chunks, m.nk) == (0, 0)
                    continue
                n_chunks = L // c
                target = max(c, math.ceil(L * ratio))
                nk = min(n_chunks, ((target + c - 1) // c * c) // c)
                assert (m.n_chunks, m.nk) == (n_chunks, max(1, nk))
                assert m.n_dense == max(1, int(m.nk * 0.3))
                assert np.array_equal(m.skipped, np.arange(n_chunks * c, L))
