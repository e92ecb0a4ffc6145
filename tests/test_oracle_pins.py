"""Pins the CPU oracle (oracle/vdx_oracle.c) before the parity tests trust it.

The reference has no golden vectors for its sampler (its only tests are the
invariants in testbed/UTest.Sampler.pas).  Each oracle function is therefore
checked against what fixes it independently:
  * published known answers (SplitMix64, xoshiro256**, Philox via numpy),
  * closed forms (mod-2^64 arithmetic, uniform rows, argmax),
  * brute-force restatements on tiny inputs (tests/npref.py),
  * the reference's own invariant tests, ported.
Each check is chosen so that a plausible slip (wrong shift, dropped term,
swapped comparison, wrong tie rule) fails it.
"""
import itertools
import json
import os

import numpy as np
import pytest

import npref
from oracle import vdx_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ---------------------------------------------------------------- PRNG ----
def test_splitmix64_known_answer():
    # SplitMix64 from state 0: first output 0xE220A8397B1DCDAF (Steele, Lea,
    # Flood; the value every SplitMix64 implementation is checked against).
    assert O.splitmix64_stream(0, 1)[0] == 0xE220A8397B1DCDAF


@pytest.mark.parametrize("seed", [0, 1, 42, 2**63, 2**64 - 1, 0x123456789ABCDEF])
def test_splitmix64_matches_restatement(seed):
    s = seed
    want = []
    for _ in range(64):
        s, z = npref.splitmix64(s)
        want.append(z)
    assert O.splitmix64_stream(seed, 64) == want


def test_wrap_arithmetic_is_mod_2_64():
    # WrapMul/WrapAdd (Sampler.pas:160-190) are plain mod-2^64 arithmetic.
    rng = np.random.default_rng(5)
    L = O.lib()
    vals = [0, 1, 2**32 - 1, 2**32, 2**63, 2**64 - 1] + [int(x) for x in rng.integers(0, 2**63, 200)] \
        + [int(x) | (1 << 63) for x in rng.integers(0, 2**63, 200)]
    for a, b in itertools.product(vals[:40], vals[:40]):
        assert L.vdxo_wrap_mul(a, b) == (a * b) & npref.MASK64
        assert L.vdxo_wrap_add(a, b) == (a + b) & npref.MASK64
    for a, b in zip(vals, reversed(vals)):
        assert L.vdxo_wrap_mul(a, b) == (a * b) & npref.MASK64


def test_xoshiro_known_answer():
    # xoshiro256** from state {1,2,3,4}: r0 = rotl(2*5,7)*9 = 11520; after one
    # step s1 = 0 so r1 = 0; then s1 = 262149 so r2 = 262149*5*128*9.
    out = O.xoshiro_stream([1, 2, 3, 4], 3)
    assert out == [11520, 0, 1509978240]


@pytest.mark.parametrize("seed", [1, 42, 2**63 + 5, 2**64 - 1, 1000])
def test_xoshiro_matches_restatement(seed):
    st = npref.seed(seed)
    assert O.seed_state(seed) == st
    want = [npref.xoshiro_next(st) for _ in range(2000)]
    assert O.xoshiro_stream(O.seed_state(seed), 2000) == want


def test_next_float_resolution():
    # NextFloat = (x shr 40) / 2^24: a multiple of 2^-24 in [0, 1).
    L = O.lib()
    for x in [0, 1 << 40, (1 << 64) - 1, 0x8000000000000000]:
        u = L.vdxo_u24(x)
        assert u == (x >> 40) / 16777216.0
        assert 0.0 <= u < 1.0


def test_philox4x64_10_matches_numpy():
    # numpy.random.Philox is Philox4x64-10; it increments the 256-bit counter
    # before generating each block of four words.
    rng = np.random.default_rng(11)
    for _ in range(50):
        key = [int(x) for x in rng.integers(0, 2**63, 2, dtype=np.uint64)]
        key[1] |= int(rng.integers(0, 2)) << 63
        ctr = [int(x) for x in rng.integers(0, 2**63, 4, dtype=np.uint64)]
        bg = np.random.Philox(key=np.array(key, dtype=np.uint64),
                              counter=np.array(ctr, dtype=np.uint64))
        want = [int(x) for x in bg.random_raw(4)]
        c = sum(v << (64 * i) for i, v in enumerate(ctr)) + 1
        c1 = [(c >> (64 * i)) & npref.MASK64 for i in range(4)]
        assert O.philox4x64_10(c1, key) == want


def test_philox_golden_fixture():
    g = _golden("philox4x64_10.json")
    for case in g["cases"]:
        assert O.philox4x64_10(case["ctr"], case["key"]) == case["out"]


def test_philox_uniform_layout():
    # Uniform for (seed, row, step) = top 24 bits of word 0 at counter
    # {step, row, 0, 0}, key {seed, 0}.
    w = O.philox4x64_10([7, 3, 0, 0], [99, 0])[0]
    assert O.philox_uniform(99, 3, 7) == (w >> 40) / 16777216.0


# ------------------------------------------------------------- penalty ----
def test_penalty_bruteforce():
    rng = np.random.default_rng(3)
    for trial in range(200):
        V = int(rng.integers(1, 40))
        L = (rng.standard_normal(V) * 3).astype(np.float32)
        L[rng.integers(0, V)] = 0.0
        H = rng.integers(-3, V + 3, int(rng.integers(0, 30))).astype(np.int32)
        p = float(np.float32(rng.choice([1.1, 2.0, 0.7, -1.5, 1.0])))
        want = npref.penalty(L, H, p)
        got = L.copy()
        if p != 1.0:
            O.lib().vdxo_apply_penalty(O._fp(got), V, O._ip(H), len(H), p)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), trial


def test_penalty_once_per_occurrence_closed_form():
    L = np.array([3.0, -2.0, 5.0], dtype=np.float32)
    H = np.array([0, 0, 0, 1, 1, 7, -1], dtype=np.int32)
    O.lib().vdxo_apply_penalty(O._fp(L), 3, O._ip(H), len(H), 1.1)
    p = np.float32(1.1)
    assert L[0] == np.float32(np.float32(np.float32(3.0) / p) / p) / p
    assert L[1] == np.float32(np.float32(-2.0) * p) * p
    assert L[2] == 5.0


# -------------------------------------------------------------- greedy ----
def test_greedy_first_index_of_max():
    rng = np.random.default_rng(4)
    cfg = O.make_config(temperature=0.0)
    for _ in range(100):
        V = int(rng.integers(1, 3000))
        L = rng.integers(-5, 5, V).astype(np.float32)  # many exact ties
        assert O.process_row(L.copy(), cfg, 0.5) == int(np.argmax(L))
    L = np.array([np.nan, 1.0, 2.0], dtype=np.float32)
    assert O.process_row(L, cfg, 0.5) == 0  # NaN at 0 absorbs the strict '>' scan
    L = np.array([1.0, np.nan, 2.0], dtype=np.float32)
    assert O.process_row(L, cfg, 0.5) == 2
    L = np.array([-0.0, 0.0], dtype=np.float32)
    assert O.process_row(L, cfg, 0.5) == 0  # -0 == +0: lowest index wins


# ----------------------------------------------------- top-K min-buffer ----
def test_topk_boundary_tie_example():
    # [5,1,5,7], K=2 keeps indices {3,2} in slots [3,2]: index 0 (value 5) is
    # evicted by index 3 because slot 0 is the first slot holding the minimum.
    L = np.array([5, 1, 5, 7], dtype=np.float32)
    cfg = O.make_config(temperature=1.0, top_k=2)
    _, tr = O.process_row(L, cfg, 0.0, trace=True)
    assert list(tr.slot_idx[:2]) == [3, 2]
    assert list(tr.slot_val[:2]) == [7.0, 5.0]


def test_topk_slots_bruteforce_small():
    cfg_base = dict(temperature=1.0, top_p=1.0)
    n = 0
    for V in range(2, 7):
        for vals in itertools.product([0.0, 1.0, 2.0], repeat=V):
            L = np.array(vals, dtype=np.float32)
            for K in range(1, V):
                cfg = O.make_config(top_k=K, **cfg_base)
                _, tr = O.process_row(L.copy(), cfg, 0.5, trace=True)
                sv, si, M = npref.topk_slots(L, K)
                assert list(tr.slot_idx[:K]) == si, (vals, K)
                assert list(tr.slot_val[:K]) == [float(x) for x in sv]
                assert tr.max_logit == M
                n += 1
    assert n > 1000


def test_topk_distinct_set_is_argsort():
    rng = np.random.default_rng(8)
    for _ in range(50):
        V = int(rng.integers(70, 5000))
        K = int(rng.integers(1, 65))
        L = rng.permutation(V).astype(np.float32) * np.float32(0.01)
        cfg = O.make_config(temperature=1.0, top_k=K)
        _, tr = O.process_row(L.copy(), cfg, 0.3, trace=True)
        assert sorted(tr.slot_idx[:K]) == sorted(np.argsort(-L, kind="stable")[:K].tolist())


@pytest.mark.parametrize("top_p,min_p,T", [(1.0, 0.0, 1.0), (0.95, 0.0, 1.0), (0.9, 0.05, 0.7),
                                           (0.5, 0.0, 2.0), (1.0, 0.2, 0.8), (0.0, 0.0, 1.0)])
def test_topk_tail_matches_restatement(top_p, min_p, T):
    rng = np.random.default_rng(int(top_p * 100 + min_p * 1000 + T * 7))
    for trial in range(60):
        V = int(rng.integers(10, 2000))
        K = int(rng.integers(1, min(V, 65)))
        L = (rng.standard_normal(V) * 3).astype(np.float32)
        if trial % 3 == 0:
            L = np.round(L).astype(np.float32)  # ties
        u = np.float32(rng.integers(0, 2**24) / 2**24)
        cfg = O.make_config(temperature=T, top_k=K, top_p=top_p, min_p=min_p)
        tok, tr = O.process_row(L.copy(), cfg, float(u), trace=True)
        sv, si, M = npref.topk_slots(L, K)
        inv_t = np.float32(np.float32(1.0) / np.float32(T))
        wtok, widx, wq, wS = npref.topk_tail(sv, si, M, inv_t, top_p, min_p, u)
        assert tok == wtok, trial
        assert list(tr.order_idx[:K]) == widx
        assert np.array_equal(np.array(tr.order_q[:K], dtype=np.float32), wq)
        assert tr.sum_final == wS


def test_topk_uniform_closed_form():
    # Equal logits never enter the buffer after the first K (strict '>'), so the
    # slots hold 0..K-1, every q is 1 and S = K: the draw returns floor(u*K).
    K, V = 64, 1000
    L = np.full(V, 0.25, dtype=np.float32)
    for k in range(0, 2**24, 2**24 // 97):
        u = k / 2**24
        tok = O.process_row(L.copy(), O.make_config(temperature=1.0, top_k=K), u)
        assert tok == int(np.floor(np.float64(np.float32(u)) * K))


@pytest.mark.parametrize("top_p", [0.5, 0.25, 0.95, 0.3, 0.999, 1e-9])
def test_topk_top_p_uniform_closed_form(top_p):
    # Equal logits: slots hold 0..K-1, every q = 1, S = K.  The stable sort
    # keeps slot order; the cut keeps q while C < target = TopP * K, i.e. the
    # n = ceil(target) entries C = 0 .. n-1 (the crossing entry included);
    # S' = n and the draw returns floor(u * n).  "C <= target", dropping the
    # crossing entry, or a target on S' instead of S all fail here.
    K, V = 64, 700
    L = np.full(V, -1.75, dtype=np.float32)
    target = np.float64(np.float32(top_p)) * K
    n = int(np.ceil(target))
    for k in range(0, 2**24, 2**24 // 61):
        u = k / 2**24
        tok, tr = O.process_row(L.copy(), O.make_config(temperature=0.9, top_k=K, top_p=top_p), u, trace=True)
        assert tr.sum_final == n
        assert tok == int(np.floor(np.float64(np.float32(u)) * n)), (top_p, u)


@pytest.mark.parametrize("top_p", [1.0, 0.6])
def test_topk_min_p_two_level_closed_form(top_p):
    # K = 64 slots over a row of zeros with 10 logits of 5.0 at indices >= K:
    # each 5.0 enters and evicts the first strict-minimum slot, so they take
    # slots 0..9 in index order; slots 10..63 keep indices 10..63 (value 0).
    # q = 1 for the 5.0 entries, qB = fl32(exp(-5 invT)) for the rest.
    K, V, T = 64, 5000, 1.25
    rng = np.random.default_rng(31)
    hot = np.sort(rng.choice(np.arange(K, V), 10, replace=False))
    L = np.zeros(V, dtype=np.float32)
    L[hot] = 5.0
    inv_t = np.float32(np.float32(1.0) / np.float32(T))
    qb = np.float32(np.exp(np.float64(-5.0) * np.float64(inv_t)))
    us = [k / 2**24 for k in range(0, 2**24, 2**24 // 53)] + [1 - 2**-24]
    # (a) MinP above qB: every q < thr = fl32(1 * MinP) is zeroed, S = 10;
    #     Top-P keeps n = ceil(TopP * 10) of the equal q in slot order
    n = int(np.ceil(np.float64(np.float32(top_p)) * 10))
    for u in us:
        tok = O.process_row(L.copy(), O.make_config(temperature=T, top_k=K, top_p=top_p,
                                                    min_p=float(qb) * 1.5), u)
        assert tok == hot[int(np.floor(np.float64(np.float32(u)) * n))], u
    # (b) MinP = qB exactly: q < thr is strict, so nothing is zeroed and
    #     S = 10 + 54 qB exactly (every partial sum fits in 53 bits); with
    #     TopP = 1 the draw walks the slots: hot[floor(t)] while t < 10,
    #     else index 10 + j for the first j with 10 + (j + 1) qB > t
    if top_p == 1.0:
        S = 10.0 + 54.0 * np.float64(qb)
        for u in us:
            tok, tr = O.process_row(L.copy(), O.make_config(temperature=T, top_k=K, min_p=float(qb)), u,
                                    trace=True)
            assert tr.sum_final == S
            t = np.float64(np.float32(u)) * S
            if t < 10.0:
                want = hot[int(np.floor(t))]
            else:
                j = 0
                while not (10.0 + (j + 1) * np.float64(qb) > t):
                    j += 1
                want = 10 + j
            assert tok == want, u


# ------------------------------------------------------------ full path ----
@pytest.mark.parametrize("min_p,T", [(0.0, 1.0), (0.0, 0.7), (0.05, 1.3)])
def test_full_path_matches_restatement(min_p, T):
    rng = np.random.default_rng(int(T * 10 + min_p * 100))
    for trial in range(20):
        V = int(rng.integers(2, 30000))
        L = (rng.standard_normal(V) * 3).astype(np.float32)
        u = np.float32(rng.integers(0, 2**24) / 2**24)
        cfg = O.make_config(temperature=T, top_k=0, min_p=min_p)
        tok, tr = O.process_row(L.copy(), cfg, float(u), trace=True)
        inv_t = np.float32(np.float32(1.0) / np.float32(T))
        wtok, q, S, t, c = npref.full_path(L, inv_t, min_p, u)
        assert tok == wtok
        assert tr.sum_final == S
        assert tr.target == t


def test_full_path_uniform_closed_form():
    # All q = 1, S = V exactly, t = u*V: the first i with i+1 > t is floor(u*V).
    V = 262144
    L = np.full(V, -3.5, dtype=np.float32)
    for k in [0, 1, 12345, 2**23, 2**24 - 1]:
        u = k / 2**24
        tok = O.process_row(L.copy(), O.make_config(temperature=0.7), u)
        assert tok == int(np.floor(np.float64(np.float32(u)) * V))


def test_full_path_ignores_top_p():
    # TopP is not applied when TopK = 0 (Sampler.pas:461-527).
    rng = np.random.default_rng(2)
    L = (rng.standard_normal(5000) * 2).astype(np.float32)
    for u in [0.1, 0.5, 0.99]:
        a = O.process_row(L.copy(), O.make_config(temperature=0.7, top_k=0, top_p=0.9), u)
        b = O.process_row(L.copy(), O.make_config(temperature=0.7, top_k=0, top_p=1.0), u)
        assert a == b


def test_full_path_nan_falls_back_to_last():
    L = np.array([0.0, np.nan, 1.0, 2.0], dtype=np.float32)
    assert O.process_row(L, O.make_config(temperature=1.0), 0.1) == 3


# ------------------------------------- reference invariants (UTest.Sampler) --
def test_ref_defaults():
    # testbed/UTest.Sampler.pas:68-92
    c = O.Sampler().get_config()
    assert (c.temperature, c.top_k, c.top_p, c.min_p, c.repeat_penalty, c.repeat_window, c.seed) \
        == (0.0, 0, 1.0, 0.0, 1.0, 64, 0)


def test_ref_greedy():
    # testbed/UTest.Sampler.pas:99-133
    s = O.Sampler()
    s.set_config(O.make_config(temperature=0.0))
    L = np.full(10, 0.1, dtype=np.float32)
    L[7] = 5.0
    assert s.process(L) == 7
    L[7] = 0.1
    L[2] = 9.9
    assert s.process(L) == 2


def test_ref_determinism():
    # testbed/UTest.Sampler.pas:141-193
    L = (np.arange(10) * 0.25).astype(np.float32)
    seqs = []
    for _ in range(2):
        s = O.Sampler()
        s.set_config(O.make_config(temperature=1.0, seed=42))
        seqs.append([s.process(L) for _ in range(50)])
    assert seqs[0] == seqs[1]


def test_ref_topk_bound():
    # testbed/UTest.Sampler.pas:200-248
    L = np.zeros(10, dtype=np.float32)
    L[[1, 4, 8]] = 10.0
    s = O.Sampler()
    s.set_config(O.make_config(temperature=1.0, top_k=3, seed=42))
    assert all(s.process(L) in (1, 4, 8) for _ in range(200))


def test_ref_repeat_penalty():
    # testbed/UTest.Sampler.pas:259-327
    L = np.ones(10, dtype=np.float32)
    hits = []
    for rp in (1.0, 2.0):
        s = O.Sampler()
        s.set_config(O.make_config(temperature=1.0, repeat_penalty=rp, seed=42))
        if rp != 1.0:
            s.add_to_history(3)
        hits.append(sum(s.process(L.copy()) == 3 for _ in range(200)))
    assert hits[1] < hits[0]
    assert hits[0] > 5


def test_history_ring_and_reseed():
    # AddToHistory / ResetHistory / SetConfig (Sampler.pas:132-150, 530-549)
    s = O.Sampler()
    s.set_config(O.make_config(temperature=1.0, repeat_window=3, seed=7))
    for t in [10, 11, 12, 13]:
        s.add_to_history(t)
    h, pos = s.history()
    assert h == [13, 11, 12] and pos == 1
    st0 = s.rng_state()
    L = np.zeros(5, dtype=np.float32)
    s.process(L)
    assert s.rng_state() != st0
    s.reset_history()
    assert s.history() == ([], 0)
    assert s.rng_state() == npref.seed(7)
    s.set_config(O.make_config(temperature=1.0, repeat_window=3, seed=-5))
    st = s.rng_state()
    s.process(L)
    s.reset_history()  # Seed < 0 is not reseeded by ResetHistory
    assert s.rng_state() != st
    s.set_config(O.make_config(temperature=1.0, repeat_window=4, seed=-5))
    assert s.history() == ([], 0)  # window change clears the ring


def test_stateful_process_uses_one_draw_per_call():
    s = O.Sampler()
    s.set_config(O.make_config(temperature=0.8, top_k=5, top_p=0.9, seed=123))
    st = npref.seed(123)
    rng = np.random.default_rng(0)
    for _ in range(20):
        L = rng.standard_normal(100).astype(np.float32)
        u = npref.u24(npref.xoshiro_next(st))
        want = O.process_row(L.copy(), O.make_config(temperature=0.8, top_k=5, top_p=0.9), float(u))
        assert s.process(L.copy()) == want
    g = O.Sampler()
    g.set_config(O.make_config(temperature=0.0, seed=123))
    st = g.rng_state()
    g.process(np.ones(4, dtype=np.float32))
    assert g.rng_state() == st  # greedy draws nothing


# ----------------------------------------------------------------- Q4_0 ----
def _rand_q4_0(rng, rows, in_dim):
    nb = in_dim // 32
    blk = np.zeros((rows, nb, 18), dtype=np.uint8)
    d = np.abs(rng.standard_normal((rows, nb)) * 0.02).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def test_half_to_float_matches_numpy():
    L = O.lib()
    hs = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    want = hs.view(np.float16).astype(np.float32)
    got = np.array([L.vdxo_half_to_float(int(h)) for h in hs[::7]], dtype=np.float32)
    w = want[::7]
    ok = (got == w) | (np.isnan(got) & np.isnan(w))
    assert ok.all()


def test_q4_0_matvec_against_dequant():
    rng = np.random.default_rng(9)
    rows, in_dim = 64, 2560
    w = _rand_q4_0(rng, rows, in_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    got = O.matvec_q4_0(w, x, in_dim, rows)
    W = npref.q4_0_dequant(w, in_dim, rows).astype(np.float64)
    want = W @ x.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4)
    # the shader's order: per-lane strided fp32 partials, then the tree
    Wf = npref.q4_0_dequant(w, in_dim, rows)
    part = np.zeros((rows, 64), dtype=np.float32)
    for e in range(in_dim):
        part[:, e % 64] = (part[:, e % 64] + (Wf[:, e] * x[e]).astype(np.float32)).astype(np.float32)
    s = 32
    while s:
        part[:, :s] = (part[:, :s] + part[:, s:2 * s]).astype(np.float32)
        s //= 2
    assert np.array_equal(got, part[:, 0])


def _exact_q4_0(rng, rows, in_dim):
    """Q4_0 rows whose scales are 2^-4 or 2^-3 and hidden values multiples of
    2^-3 in [-4, 4): every product and partial sum is an exact fp32 value, so
    any summation order gives the exact (float64) result."""
    nb = in_dim // 32
    blk = np.zeros((rows, nb, 18), dtype=np.uint8)
    d = np.where(rng.random((rows, nb)) < 0.5, 2.0 ** -4, 2.0 ** -3).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    x = (rng.integers(-32, 32, in_dim) / 8.0).astype(np.float32)
    return blk.reshape(-1), x


def test_q4_0_both_orders_exact_on_exact_inputs():
    # closed form: both restatements (the shader's order and the kernel's
    # blocked order) equal the exact dot product of the dequantised rows
    rng = np.random.default_rng(21)
    for in_dim in (256, 2560):
        rows = 40
        w, x = _exact_q4_0(rng, rows, in_dim)
        want = npref.q4_0_dequant(w, in_dim, rows).astype(np.float64) @ x.astype(np.float64)
        assert np.array_equal(O.matvec_q4_0(w, x, in_dim, rows).astype(np.float64), want)
        assert np.array_equal(O.matvec_q4_0_blocked(w, x, in_dim, rows).astype(np.float64), want)
        assert np.array_equal(O.matvec_q4_0_mt(w, x, in_dim, rows, True, 3).astype(np.float64), want)
        assert np.array_equal(O.matvec_q4_0_mt(w, x, in_dim, rows, False, 3).astype(np.float64), want)


def test_q4_0_blocked_nibble_order_is_pinned():
    # a single non-zero nibble at each element position in turn: only the
    # documented element order (low nibbles of qs[0..15], then high nibbles)
    # reproduces x[e] * (q - 8) * d at position e
    in_dim, rows = 256, 1
    x = (np.arange(in_dim) + 1).astype(np.float32)
    for e in (0, 5, 15, 16, 17, 31, 32, 47, 200):
        blk = np.zeros((in_dim // 32, 18), dtype=np.uint8)
        blk[:, 0:2] = np.array([1.0], dtype=np.float16).view(np.uint8)
        blk[:, 2:] = 0x88  # q = 8 everywhere: weight 0
        k, i = divmod(e, 32)
        b = blk[k, 2 + (i & 15)]
        blk[k, 2 + (i & 15)] = (b & 0xF0) | 0x0B if i < 16 else (b & 0x0F) | 0xB0  # q = 11: weight 3
        got = O.matvec_q4_0_blocked(blk.reshape(-1), x, in_dim, rows)[0]
        assert got == np.float32(3.0 * (e + 1)), (e, got)
        assert O.matvec_q4_0(blk.reshape(-1), x, in_dim, rows)[0] == got


def test_q4_0_blocked_within_fp32_error_bound():
    # realistic inputs (config 5: scales |N(0, 0.02)|, hidden N(0,1)): the
    # blocked order and the shader's order each stay within the standard
    # summation bound of the exact (float64) result
    rng = np.random.default_rng(22)
    rows, in_dim = 256, 2560
    w = _rand_q4_0(rng, rows, in_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    W = npref.q4_0_dequant(w, in_dim, rows).astype(np.float64)
    exact = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    u = 2.0 ** -24
    blocked = O.matvec_q4_0_blocked(w, x, in_dim, rows).astype(np.float64)
    shader = O.matvec_q4_0(w, x, in_dim, rows).astype(np.float64)
    assert (np.abs(blocked - exact) <= (32 + in_dim // 32 + 1) * u * mag).all()
    assert (np.abs(shader - exact) <= (in_dim // 64 + 6 + 1) * u * mag).all()
    # the two orders agree far inside the bound on typical rows
    assert np.median(np.abs(blocked - shader) / mag) < 1e-7


# ---- Q8_0 / F16 lm_head and the output RMSNorm (matvec_q8_0.comp,
# ---- matvec_f16.comp, rmsnorm_copy.comp) ---------------------------------------
def _rand_q8_0(rng, rows, in_dim, exact=False):
    nb = in_dim // 32
    blk = np.zeros((rows, nb, 34), dtype=np.uint8)
    if exact:
        d = np.where(rng.random((rows, nb)) < 0.5, 2.0 ** -4, 2.0 ** -3).astype(np.float16)
    else:
        d = np.abs(rng.standard_normal((rows, nb)) * 0.02).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, nb, 32), dtype=np.uint8)
    return blk.reshape(-1)


def _rand_f16(rng, rows, in_dim, exact=False):
    if exact:  # multiples of 1/8 in [-8, 8)
        w = (rng.integers(-64, 64, (rows, in_dim)) / 8.0).astype(np.float16)
    else:
        w = (rng.standard_normal((rows, in_dim)) * 0.05).astype(np.float16)
    return w.view(np.uint8).reshape(-1)


@pytest.mark.parametrize("wtype", [O.TENSOR_Q8_0, O.TENSOR_F16])
def test_q8_f16_both_orders_exact_on_exact_inputs(wtype):
    # closed form: with power-of-two scales, weights and hidden values on a
    # coarse grid every product and partial sum is exact, so both
    # restatements equal the float64 dot product of the dequantised rows
    rng = np.random.default_rng(31 + wtype)
    for in_dim in (256, 2560):
        rows = 24
        if wtype == O.TENSOR_Q8_0:
            w = _rand_q8_0(rng, rows, in_dim, exact=True)
            W = npref.q8_0_dequant(w, in_dim, rows).astype(np.float64)
            x = (rng.integers(-4, 4, in_dim) / 8.0).astype(np.float32)
        else:
            w = _rand_f16(rng, rows, in_dim, exact=True)
            W = npref.f16_dequant(w, in_dim, rows).astype(np.float64)
            x = (rng.integers(-8, 8, in_dim) / 8.0).astype(np.float32)
        want = W @ x.astype(np.float64)
        for blocked in (False, True):
            assert np.array_equal(O.matvec(w, wtype, x, in_dim, rows, blocked).astype(np.float64), want)
            assert np.array_equal(O.matvec(w, wtype, x, in_dim, rows, blocked, threads=3).astype(np.float64),
                                  want)


def test_q8_0_byte_order_is_pinned():
    # one non-zero int8 at each element position in turn: only the documented
    # layout (scale in bytes 0-1, element i in byte 2 + i, signed) reproduces
    # x[e] * q * d at position e
    in_dim = 256
    x = (np.arange(in_dim) + 1).astype(np.float32)
    for e in (0, 1, 31, 32, 33, 100, 255):
        blk = np.zeros((in_dim // 32, 34), dtype=np.uint8)
        blk[:, 0:2] = np.array([2.0], dtype=np.float16).view(np.uint8)
        k, i = divmod(e, 32)
        blk[k, 2 + i] = np.array([-3], dtype=np.int8).view(np.uint8)[0]
        for blocked in (False, True):
            got = O.matvec(blk.reshape(-1), O.TENSOR_Q8_0, x, in_dim, 1, blocked)[0]
            assert got == np.float32(-6.0 * (e + 1))


def test_q8_f16_within_fp32_error_bound():
    rng = np.random.default_rng(33)
    rows, in_dim = 128, 2560
    x = rng.standard_normal(in_dim).astype(np.float32)
    u = 2.0 ** -24
    for wtype, w, deq in ((O.TENSOR_Q8_0, _rand_q8_0(rng, rows, in_dim), npref.q8_0_dequant),
                          (O.TENSOR_F16, _rand_f16(rng, rows, in_dim), npref.f16_dequant)):
        W = deq(w, in_dim, rows).astype(np.float64)
        exact = W @ x.astype(np.float64)
        mag = np.abs(W) @ np.abs(x.astype(np.float64))
        for blocked in (False, True):
            got = O.matvec(w, wtype, x, in_dim, rows, blocked).astype(np.float64)
            assert (np.abs(got - exact) <= (in_dim // 32 + 260) * u * mag).all(), (wtype, blocked)


def test_rmsnorm_closed_forms():
    # constant rows: every partial sum is exact, so inv_rms is the correctly
    # rounded 1/sqrt(c^2 + eps); c = 1/2, eps = 0 gives exactly 2 and the
    # output is the weight itself
    dim = 2560
    w = np.random.default_rng(34).standard_normal(dim).astype(np.float32)
    h = np.full(dim, 0.5, dtype=np.float32)
    assert np.array_equal(O.rmsnorm(h, w, 0.0), w)
    for c, eps in ((3.0, 1e-6), (0.125, 1e-6), (1.0, 0.5)):
        h = np.full(dim, c, dtype=np.float32)
        inv = np.float32(1.0) / np.sqrt(np.float32(np.float32(c * c) + np.float32(eps)))
        want = (h * inv) * w
        assert np.array_equal(O.rmsnorm(h, w, eps), want)


def test_rmsnorm_against_float64():
    rng = np.random.default_rng(35)
    for dim in (256, 2560, 1000):
        h = (rng.standard_normal(dim) * 10.0).astype(np.float32)
        w = rng.standard_normal(dim).astype(np.float32)
        got = O.rmsnorm(h, w, 1e-6).astype(np.float64)
        want = h.astype(np.float64) / np.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-6) * w
        assert np.allclose(got, want, rtol=2e-6, atol=0), np.abs(got - want).max()
