"""GPU parity of the RaBitQ 1-bit encode / estimate / search against the CPU
oracle: codes, factors, estimates, candidate sets, reranked order and exact
scores are all bit-exact."""
import numpy as np
import pytest
import torch

from oracle import rabitq as orq
from oracle.numerics import f16_bits
from tests.helpers import from_torch

pytestmark = pytest.mark.gpu


def _f16(a_bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a_bits.view(np.int16)).view(torch.float16).cuda()


def _bits(t: torch.Tensor) -> np.ndarray:
    return from_torch(t.view(torch.int16)).view(np.uint16)


def _signs(seed=42):
    s = orq.srht_signs(seed)
    return s, torch.from_numpy(s).cuda()


def test_encode_bit_exact(rng):
    s_np, s_t = _signs(7)
    keys = np.concatenate([
        orq.clustered_unit_keys(rng, 3000, 16),
        f16_bits((rng.standard_normal((500, 128)) * 30).astype(np.float32)),
        np.zeros((2, 128), np.uint16),                                  # zero vector: corr 0
        f16_bits(np.full((1, 128), 60000.0, np.float32)),               # near fp16 max
        f16_bits(np.where(np.arange(128) == 5, 1.0, 0.0)[None].astype(np.float32)),
    ])
    codes, fac = orq.encode(keys, s_np)
    gc, gf = __import__("zoomkv_revision_amd.rabitq", fromlist=["x"]).rabitq_encode(_f16(keys), s_t)
    assert np.array_equal(from_torch(gc), codes)
    assert np.array_equal(_bits(gf), fac)


def test_encode_strided_rows(rng):
    from zoomkv_revision_amd.rabitq import rabitq_encode
    s_np, s_t = _signs(3)
    big = orq.clustered_unit_keys(rng, 2 * 700, 8).reshape(700, 256)   # rows of 256, use first 128
    t = _f16(big)[:, :128]
    gc, gf = rabitq_encode(t, s_t)
    codes, fac = orq.encode(np.ascontiguousarray(big[:, :128]), s_np)
    assert np.array_equal(from_torch(gc), codes) and np.array_equal(_bits(gf), fac)


def test_estimate_bit_exact(rng):
    from zoomkv_revision_amd.rabitq import rabitq_encode, rabitq_estimate
    s_np, s_t = _signs()
    keys = orq.clustered_unit_keys(rng, 5000, 32)
    qs = orq.clustered_unit_keys(rng, 7, 32)
    ck, fk = orq.encode(keys, s_np)
    cq, fq = orq.encode(qs, s_np)
    got = rabitq_estimate(*rabitq_encode(_f16(qs), s_t), *rabitq_encode(_f16(keys), s_t))
    ref = orq.estimate(cq, fq, ck, fk)
    assert np.array_equal(from_torch(got).view(np.uint32), ref.view(np.uint32))


def _check_search(rng, P, Q, N, topk, seed=42, dup=None):
    from zoomkv_revision_amd.rabitq import rabitq_encode, rabitq_search
    s_np, s_t = _signs(seed)
    keys = [orq.clustered_unit_keys(rng, N if dup is None else dup, 16) for _ in range(P)]
    if dup is not None:               # many identical keys: ties everywhere
        keys = [k[rng.integers(0, dup, size=N)] for k in keys]
    qs = [orq.clustered_unit_keys(rng, Q, 16) for _ in range(P)]
    kt = _f16(np.stack(keys))
    codes, fac = rabitq_encode(kt, s_t)
    cand, fidx, fsc = rabitq_search(_f16(np.stack(qs)), kt, codes, fac, s_t, topk)
    cand, fidx, fsc = from_torch(cand), from_torch(fidx), from_torch(fsc)
    for p in range(P):
        ck, fk = orq.encode(keys[p], s_np)
        rc, ri, rs = orq.search(qs[p], keys[p], ck, fk, s_np, topk)
        assert np.array_equal(cand[p], rc), f"pool {p}: candidate set"
        assert np.array_equal(fidx[p], ri), f"pool {p}: reranked order"
        assert np.array_equal(fsc[p].view(np.uint32), rs.view(np.uint32)), f"pool {p}: exact scores"


@pytest.mark.parametrize("P,Q,N,topk", [
    (1, 4, 20000, 256),        # 3 slices, last one partial
    (2, 3, 8192, 256),         # exactly one slice
    (1, 2, 8192 + 100, 256),   # last slice shorter than topk: padded candidates
    (1, 3, 300, 256),          # one slice, radix path
    (1, 2, 256, 256),          # topk == n
    (3, 2, 5000, 1),           # topk 1
    (1, 2, 40000, 100),        # non power-of-two topk
    (1, 1, 4000, 1000),        # topk near the limit
])
def test_search_bit_exact(rng, P, Q, N, topk):
    _check_search(rng, P, Q, N, topk)


def test_search_ties_go_to_lower_index(rng):
    _check_search(rng, 1, 4, 30000, 256, dup=40)


@pytest.mark.parametrize("P,Q,N,topk", [
    (1, 2, 65536, 1024),       # 8 slices x topk 1024 = the 8192-candidate limit
    (1, 3, 3000, 256),
    (2, 2, 2048, 300),
])
def test_search_more_sizes(rng, P, Q, N, topk):
    _check_search(rng, P, Q, N, topk)


def test_search_all_keys_equal(rng):
    """Every key identical: every estimate ties, and the top-k are the lowest
    indices."""
    _check_search(rng, 1, 2, 20000, 256, dup=1)


def test_search_few_planted_winners(rng):
    """The query itself planted at 32 spread positions: those 32 keys lead the
    candidates, the other 224 come from the clustered rest."""
    from zoomkv_revision_amd.rabitq import rabitq_encode, rabitq_search
    s_np, s_t = _signs()
    n, topk = 50000, 256
    keys = orq.clustered_unit_keys(rng, n, 16)
    qs = orq.clustered_unit_keys(rng, 1, 16)
    keys[[s * n // 2048 for s in range(32)]] = qs[0]
    kt = _f16(keys)
    codes, fac = rabitq_encode(kt, s_t)
    cand, fidx, fsc = (from_torch(t) for t in rabitq_search(_f16(qs), kt, codes, fac, s_t, topk))
    ck, fk = orq.encode(keys, s_np)
    rc, ri, rs = orq.search(qs, keys, ck, fk, s_np, topk)
    assert set([s * n // 2048 for s in range(32)]) <= set(cand[0].tolist())
    assert np.array_equal(cand, rc) and np.array_equal(fidx, ri)
    assert np.array_equal(fsc.view(np.uint32), rs.view(np.uint32))


def test_search_c4_full_size(rng):
    """131072 clustered unit keys, 64 queries, top-256;
    8 of the 64 queries checked against the oracle, all 64 against invariants."""
    from zoomkv_revision_amd.rabitq import rabitq_encode, rabitq_search
    s_np, s_t = _signs()
    keys = orq.clustered_unit_keys(rng, 131072, 64)
    qs = orq.clustered_unit_keys(rng, 64, 64)
    kt = _f16(keys)
    codes, fac = rabitq_encode(kt, s_t)
    cand, fidx, fsc = (from_torch(t) for t in rabitq_search(_f16(qs), kt, codes, fac, s_t, 256))
    ck, fk = orq.encode(keys, s_np)
    assert np.array_equal(from_torch(codes), ck)
    for i in range(0, 64, 8):
        rc, ri, rs = orq.search(qs[i:i + 1], keys, ck, fk, s_np, 256)
        assert np.array_equal(cand[i], rc[0]) and np.array_equal(fidx[i], ri[0])
        assert np.array_equal(fsc[i].view(np.uint32), rs[0].view(np.uint32))
    assert np.all(np.diff(cand, axis=-1) > 0)
    assert np.all(np.diff(fsc, axis=-1) <= 0)
    assert np.array_equal(np.sort(fidx, axis=-1), cand)


def test_search_rejects_bad_sizes():
    from zoomkv_revision_amd.rabitq import rabitq_search
    s = torch.ones(128, device="cuda")
    k = torch.zeros(100, 128, dtype=torch.float16, device="cuda")
    c = torch.zeros(100, 16, dtype=torch.uint8, device="cuda")
    f = torch.zeros(100, 2, dtype=torch.float16, device="cuda")
    with pytest.raises(AssertionError):
        rabitq_search(torch.zeros(2, 128, dtype=torch.float16, device="cuda"), k, c, f, s, 101)
    big = torch.zeros(2000, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="topk"):                      # topk above 1024
        rabitq_search(torch.zeros(1, 128, dtype=torch.float16, device="cuda"), big,
                      torch.zeros(big.shape[0], 16, dtype=torch.uint8, device="cuda"),
                      torch.zeros(big.shape[0], 2, dtype=torch.float16, device="cuda"), s, 1025)
