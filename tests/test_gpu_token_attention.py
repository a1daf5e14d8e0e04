"""GPU parity of the token-list 4-bit attention (zkv_kivi4_token_attention):
Format Q tokens named by id, bf16 tail rows and a contiguous near zone in one
launch, against the float64 oracle (outputs within 2e-3, natural-log LSEs
within 1e-5 relative), over sorted, shuffled, repeated, out-of-range, empty
and maximum-length lists and several split plans; plus a list whose order is
permuted gives the same result within rounding."""
import numpy as np
import pytest
import torch

from oracle import kivi as okivi
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3
SC = 1 / np.sqrt(128)


def _setup(rng, bs, hq, kv, ng, n_rows):
    from zoomkv_revision_amd import kivi
    k = gaussian_bf16(rng, (bs, kv, ng * 32, 128), outlier_channels=1)
    v = gaussian_bf16(rng, (bs, kv, ng * 32, 128))
    cache = kivi.Kivi4Cache.allocate(bs, kv, max(ng, 1), 1)
    if ng:
        kivi.kivi4_pack(to_bf16(k), to_bf16(v), cache, 0)
    rec = okivi.quantize_kivi4(k, v) if ng else None
    rk = gaussian_bf16(rng, (bs, kv, n_rows, 128))
    rv = gaussian_bf16(rng, (bs, kv, n_rows, 128))
    q = gaussian_bf16(rng, (bs, hq, 128))
    return cache, rec, rk, rv, q


def _list(rng, kind, bs, kv, ng, n_tail, n):
    q_end = 32 * ng
    if kind == "c5":          # tokens clustered in 16-token chunks (8 per chunk) + the skipped tail
        out = []
        for _ in range(bs * kv):
            chunks = rng.choice(2 * ng, (n - n_tail) // 8, replace=False)
            t = (chunks[:, None] * 16 + np.stack([rng.choice(16, 8, replace=False) for _ in chunks])).reshape(-1)
            out.append(np.concatenate([rng.permutation(t), q_end + np.arange(n_tail)]))
        return np.array(out).reshape(bs, kv, -1)
    if kind == "sorted":
        return np.sort(np.stack([[rng.choice(q_end + n_tail, n, replace=False) for _ in range(kv)]
                                 for _ in range(bs)]), -1)
    if kind == "shuffled":
        return np.stack([[rng.choice(q_end + n_tail, n, replace=False) for _ in range(kv)] for _ in range(bs)])
    if kind == "messy":       # repeats (a sentinel id many times), negatives, ids past the tail
        t = rng.integers(-5, q_end + n_tail + 5, size=(bs, kv, n))
        t[..., : n // 3] = 0
        t[..., n // 3: n // 3 + 3] = t[..., n // 3 + 3: n // 3 + 6]
        return t
    if kind == "tail_only":
        return np.broadcast_to(q_end + np.arange(n_tail)[::-1], (bs, kv, n_tail)).copy()
    if kind == "all":
        return np.broadcast_to(np.arange(q_end + n_tail), (bs, kv, q_end + n_tail)).copy()
    raise ValueError(kind)


@pytest.mark.parametrize("bs,hq,kv,ng,n_tail,near,n,kind,splits", [
    (4, 32, 8, 80, 13, 400, 113, "c5", 0),
    (2, 32, 8, 40, 0, 300, 100, "sorted", 0),
    (2, 8, 2, 30, 20, 50, 120, "shuffled", 0),
    (2, 8, 2, 30, 9, 70, 200, "messy", 0),
    (1, 8, 2, 10, 31, 0, 31, "tail_only", 0),
    (1, 8, 2, 12, 7, 33, 391, "all", 0),
    (2, 16, 4, 50, 5, 200, 113, "c5", 1),
    (2, 16, 4, 50, 5, 200, 113, "c5", 3),
    (1, 8, 2, 64, 16, 900, 1024, "messy", 0),     # the longest list, several splits
    (1, 8, 1, 64, 16, 100, 1024, "shuffled", 1),  # the longest list in one split: raised to fit
    (1, 16, 1, 30, 9, 70, 150, "messy", 0),       # 16 query heads per KV head
    (2, 16, 2, 30, 9, 70, 150, "shuffled", 0),    # 8 query heads per KV head
    (2, 8, 2, 0, 10, 40, 10, "shuffled", 0),      # no quantized groups
])
def test_token_attention_matches_oracle(rng, bs, hq, kv, ng, n_tail, near, n, kind, splits):
    from zoomkv_revision_amd import kivi
    tail0 = 3
    near0 = tail0 + n_tail + 5
    cache, rec, rk, rv, q = _setup(rng, bs, hq, kv, ng, near0 + near + 4)
    toks = _list(rng, kind, bs, kv, ng, n_tail, n)
    print(f"[token attn] bs={bs} hq={hq} kv={kv} ng={ng} tail={n_tail} near={near} n={toks.shape[-1]} "
          f"{kind} splits={splits}", flush=True)
    out, lse = kivi.kivi4_token_attention(to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv),
                                          torch.from_numpy(toks).cuda(), tail0, n_tail, near0, near,
                                          out_dtype=torch.float32, n_splits=splits, return_lse=True)
    out, lse = from_torch(out), from_torch(lse)
    if rec is None:
        rec = okivi.Kivi4Cache(*(np.zeros((bs, kv, 0) + s, t) for s, t in
                                 (((512,), np.int32), ((16, 2, 8), np.uint16), ((512,), np.int32),
                                  ((2, 4, 4, 2, 4), np.uint16))))
    ref, ref_lse = okivi.kivi4_token_attention(q, rec, ng, rk, rv, toks, tail0, n_tail, near0, near, SC,
                                               return_lse=True)
    err = np.abs(out - ref).max()
    lerr = np.abs(lse / ref_lse - 1).max()
    assert err <= ATOL, f"max abs err {err}"
    assert lerr <= 1e-5, f"LSE rel err {lerr}"


def test_token_attention_empty_list_and_nothing_to_attend(rng):
    from zoomkv_revision_amd import kivi
    bs, hq, kv, ng = 1, 8, 2, 4
    cache, rec, rk, rv, q = _setup(rng, bs, hq, kv, ng, 64)
    none = torch.empty(bs, kv, 0, dtype=torch.int64, device="cuda")
    got = from_torch(kivi.kivi4_token_attention(to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv), none,
                                                0, 0, 10, 33, out_dtype=torch.float32))
    ref = okivi.kivi4_token_attention(q, rec, ng, rk, rv, np.zeros((bs, kv, 0), int), 0, 0, 10, 33, SC)
    assert np.abs(got - ref).max() <= ATOL
    skipped = torch.full((bs, kv, 5), -1, dtype=torch.int64, device="cuda")
    z = from_torch(kivi.kivi4_token_attention(to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv), skipped,
                                              0, 0, 10, 0, out_dtype=torch.float32))
    assert np.all(z == 0)


def test_token_attention_order_does_not_matter(rng):
    """The kernel sorts each list: a permuted list gives the same bits."""
    from zoomkv_revision_amd import kivi
    bs, hq, kv, ng, n_tail = 2, 32, 8, 60, 11
    cache, rec, rk, rv, q = _setup(rng, bs, hq, kv, ng, 600)
    toks = _list(rng, "c5", bs, kv, ng, n_tail, 100 + n_tail)
    perm = np.stack([[rng.permutation(toks[b, h]) for h in range(kv)] for b in range(bs)])
    args = lambda t: (to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv), torch.from_numpy(t).cuda(), 0,
                      n_tail, 20, 500)
    a = kivi.kivi4_token_attention(*args(toks), out_dtype=torch.float32)
    b = kivi.kivi4_token_attention(*args(perm), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_token_attention_rejects_bad_arguments(rng):
    from zoomkv_revision_amd import kivi
    from zoomkv_revision_amd._lib import ZkvError
    bs, hq, kv, ng = 1, 8, 2, 4
    cache, rec, rk, rv, q = _setup(rng, bs, hq, kv, ng, 64)
    t = torch.zeros(bs, kv, 1025, dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="1024"):
        kivi.kivi4_token_attention(to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv), t, 0, 0, 0, 10)
    t = torch.zeros(bs, kv, 4, dtype=torch.int64, device="cuda")
    with pytest.raises(ZkvError, match="outside"):
        kivi.kivi4_token_attention(to_bf16(q), cache.groups, ng, to_bf16(rk), to_bf16(rv), t, 60, 8, 0, 10)
