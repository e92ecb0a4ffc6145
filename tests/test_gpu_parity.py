"""GPU parity of libvdxsampler.so against the CPU oracle (restated TVdxSampler).

Every test calls the HIP kernels through the C ABI (ctypes) on cuda:0 and the
oracle on the same seeded inputs with the same injected per-row uniform.
Bar (bit-exact for integer work, stated tolerance for floating point):
  * argmax, top-K index sets, penalised logits: bit-exact;
  * probabilities of the final candidates: within 1e-5 relative;
  * sampled token: identical, except draws within 1e-6*S of a CDF boundary,
    which are counted and printed.
"""
import numpy as np
import pytest

from gpu_common import (canonical_topk, cfg1_logits, cfg2_logits, cfg3_inputs, cfg4_logits,
                        compare, gpu_sample, log, oracle_rows, u_stream)
from oracle import vdx_oracle as O

pytestmark = pytest.mark.gpu

ROW_GREEDY, ROW_TOPK_FAST, ROW_TOPK_REPLAY, ROW_FULL, ROW_NAN = 0x1, 0x2, 0x4, 0x8, 0x10


def _run(L, cfg, u, hist=None, label="", **kw):
    log(f"[case] {label} B={L.shape[0]} V={L.shape[1]} cfg={cfg}")
    g = gpu_sample(L.copy(), cfg, u, hist=hist, **kw)
    orc = oracle_rows(L, cfg, u, hist=hist)
    nb = compare(g, orc, cfg, label=label)
    log(f"[done] {label}: near-boundary draws {nb}/{L.shape[0]}, flags {sorted(set(g['flags'].tolist()))}")
    return g, orc, nb


# ------------------------------------------------------------- greedy ----
@pytest.mark.parametrize("B", [1, 64])
def test_cfg2_greedy_ties(B):
    rng = np.random.default_rng(1002 + B)
    L = cfg2_logits(rng, B)
    g, orc, _ = _run(L, dict(temperature=0.0), None, label=f"C2 greedy B={B}")
    for r in range(B):
        assert g["tokens"][r] == int(np.argmax(L[r]))
        assert g["flags"][r] == ROW_GREEDY


def test_greedy_nan_and_small():
    rng = np.random.default_rng(5)
    L = (rng.standard_normal((6, 1000)) * 2).astype(np.float32)
    L[0, 0] = np.nan  # absorbs the scan -> 0
    L[1, 10] = np.nan
    L[2, :] = np.nan
    L[3, [3, 700]] = 50.0
    L[4, :] = -np.inf
    L[5, 999] = 1e30
    _run(L, dict(temperature=0.0), None, label="greedy nan/ties")


# -------------------------------------------------------------- top-K ----
def test_cfg1_topk_single_row():
    rng = np.random.default_rng(1001)
    L = cfg1_logits(rng, 1)
    u = u_stream(np.random.default_rng(2001), 1)
    g, _, _ = _run(L, dict(temperature=1.0, top_k=64, top_p=0.95), u, label="C1")
    assert g["flags"][0] & ROW_TOPK_FAST


def test_cfg3_penalised_batch():
    rng = np.random.default_rng(1003)
    L, hist = cfg3_inputs(rng)
    u = u_stream(np.random.default_rng(2003), L.shape[0])
    cfg = dict(temperature=0.8, top_k=64, top_p=0.95, repeat_penalty=1.1, repeat_window=256)
    g, _, _ = _run(L, cfg, u, hist=hist, label="C3")
    assert (g["flags"] & (ROW_TOPK_FAST | ROW_TOPK_REPLAY)).all()


def test_b256_topk64_topp095():
    rng = np.random.default_rng(1006)
    L = cfg1_logits(rng, 256)
    u = u_stream(np.random.default_rng(2006), 256)
    g, _, _ = _run(L, dict(temperature=1.0, top_k=64, top_p=0.95), u, label="B256 K64 P0.95")
    assert (g["flags"] & ROW_TOPK_FAST).mean() > 0.9


@pytest.mark.parametrize("V", [10, 100, 300, 1000, 16384, 20000, 40000, 151936])
@pytest.mark.parametrize("K", [1, 3, 64])
def test_topk_shapes(V, K):
    if K >= V:
        pytest.skip("K >= V is the full path")
    rng = np.random.default_rng(V * 7 + K)
    B = 8
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    u = u_stream(rng, B)
    for P in (0.95, 1.0):
        _run(L, dict(temperature=1.0, top_k=K, top_p=P), u, label=f"topk V={V} K={K} P={P}")


@pytest.mark.parametrize("T,P,minp", [(0.7, 0.9, 0.05), (1.5, 0.5, 0.0), (1.0, 1.0, 0.1),
                                      (0.3, 0.95, 0.0), (2.0, 0.0, 0.0), (1.0, 0.95, 1.5)])
def test_topk_params(T, P, minp):
    rng = np.random.default_rng(int(T * 100 + P * 10 + minp * 1000))
    B, V = 16, 70000
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    u = u_stream(rng, B)
    _run(L, dict(temperature=T, top_k=64, top_p=P, min_p=minp), u, label=f"topk T={T} P={P} minP={minp}")


def test_topk_ties_replay():
    # integer-valued logits: ties at the K boundary and among candidates force
    # the exact min-buffer replay (the first strict-minimum slot is evicted)
    rng = np.random.default_rng(77)
    B, V = 16, 50000
    L = rng.integers(-20, 8, (B, V)).astype(np.float32)
    L[0] = 1.0  # all equal
    L[1, :10] = [5, 1, 5, 7, 5, 5, 5, 5, 5, 5]
    u = u_stream(rng, B)
    for P in (0.95, 1.0):
        g, _, _ = _run(L, dict(temperature=1.0, top_k=64, top_p=P), u, label=f"ties P={P}")
        assert (g["flags"] & ROW_TOPK_REPLAY).any()


def test_topk_boundary_example_small():
    L = np.array([[5, 1, 5, 7]], dtype=np.float32)
    g, orc, _ = _run(L, dict(temperature=1.0, top_k=2, top_p=1.0), np.array([0.25], np.float32),
                     label="[5,1,5,7] K=2")
    assert sorted(g["topk_idx"][0].tolist()) == [2, 3]


def test_topk_ref_testbed_case():
    # testbed/UTest.Sampler.pas:200-248 with injected uniforms: K=3, TopP=1, draws in slot order
    L = np.zeros((1, 10), dtype=np.float32)
    L[0, [1, 4, 8]] = 10.0
    for u in [0.0, 0.2, 0.34, 0.5, 0.67, 0.9, 0.999]:
        g, _, _ = _run(L, dict(temperature=1.0, top_k=3), np.array([u], np.float32),
                       label=f"testbed K=3 u={u}")
        assert g["tokens"][0] in (1, 4, 8)


def test_topk_nonfinite_rows():
    rng = np.random.default_rng(9)
    B, V = 8, 30000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[0, 0] = np.nan
    L[1, 500] = np.nan
    L[2, 100] = np.inf
    L[3, 5] = -np.inf
    L[4, :] = -np.inf
    L[5, 20000] = np.inf
    L[5, 20001] = -np.inf
    L[6, :64] = np.nan
    L[7, 7] = -0.0
    L[7, 8] = 0.0
    u = u_stream(rng, B)
    for P in (0.95, 1.0):
        _run(L, dict(temperature=1.0, top_k=64, top_p=P), u, label=f"nonfinite P={P}")


def test_topk_unaligned_rows():
    rng = np.random.default_rng(13)
    B, V = 8, 40001
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    u = u_stream(rng, B)
    log("[case] unaligned stride/offset")
    g = gpu_sample(L.copy(), dict(temperature=0.9, top_k=64, top_p=0.95), u, row_stride=V + 3, offset=1)
    compare(g, oracle_rows(L, dict(temperature=0.9, top_k=64, top_p=0.95), u),
            dict(), label="unaligned")


def test_topk_overflow_chunk():
    # a chunk with thousands of equal maxima overflows the candidate store
    rng = np.random.default_rng(21)
    B, V = 4, 262144
    L = (rng.standard_normal((B, V))).astype(np.float32)
    L[:, 16384:32768] = 9.0
    u = u_stream(rng, B)
    _run(L, dict(temperature=1.0, top_k=64, top_p=0.95), u, label="overflow")


def test_topk_concentrated_in_one_chunk():
    # the row's top K all in one chunk: that chunk's threshold is far above
    # every other chunk's, so fewer than K stored keys reach T = max tau_c and
    # the merge re-reads (the per-chunk quota is below K by design)
    rng = np.random.default_rng(23)
    B, V = 4, 262144
    L = (rng.standard_normal((B, V))).astype(np.float32)
    for r in range(B):
        c = 1 + 3 * r  # a different chunk per row
        L[r, c * 16384 + rng.choice(16384, 300, replace=False)] += np.float32(12.0)
    u = u_stream(rng, B)
    for K, P in ((64, 0.95), (40, 0.9), (64, 1.0)):
        _run(L, dict(temperature=1.0, top_k=K, top_p=P), u, label=f"concentrated K={K} P={P}")


# ----------------------------------------------------------- full path ----
def test_cfg4_full_vocab_b256():
    rng = np.random.default_rng(1004)
    L = cfg4_logits(rng)
    u = u_stream(np.random.default_rng(2004), 256)
    g, orc, nb = _run(L, dict(temperature=0.7, top_k=0, top_p=0.9), u, label="C4 full")
    assert (g["flags"] & ROW_FULL).all()
    assert nb <= 2


@pytest.mark.parametrize("V", [7, 1000, 16385, 100000, 262144])
@pytest.mark.parametrize("minp", [0.0, 0.02])
def test_full_path_shapes(V, minp):
    rng = np.random.default_rng(V + int(minp * 100))
    B = 8
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    u = u_stream(rng, B)
    _run(L, dict(temperature=1.0, top_k=0, min_p=minp), u, label=f"full V={V} minP={minp}")


def test_full_path_k_ge_v_and_nonfinite():
    rng = np.random.default_rng(31)
    B, V = 6, 5000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[1, 10] = np.nan
    L[2, 3] = np.inf
    L[3, :] = -np.inf
    L[4, 100] = -np.inf
    u = u_stream(rng, B)
    _run(L, dict(temperature=0.8, top_k=V), u, label="K=V full")
    _run(L, dict(temperature=0.8, top_k=-3), u, label="K<0 full")


def test_full_uniform_closed_form():
    V = 262144
    L = np.full((4, V), 0.5, dtype=np.float32)
    u = np.array([0.0, 0.25, 0.5, 1 - 2**-24], dtype=np.float32)
    g = gpu_sample(L.copy(), dict(temperature=1.0), u, topk_out=False)
    assert g["tokens"].tolist() == [int(np.floor(np.float64(x) * V)) for x in u]


# --------------------------------------------------------------- penalty ----
def test_penalty_bitexact_and_repeats():
    rng = np.random.default_rng(41)
    B, V = 8, 20000
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[:, 5] = 0.0
    hist = rng.integers(-5, V + 5, (B, 300)).astype(np.int32)
    hist[:, :40] = 5
    hist[:, 40:80] = 7
    u = u_stream(rng, B)
    for p in (1.1, 0.5, -2.0):
        for T in (0.0, 1.0):
            _run(L, dict(temperature=T, top_k=64 if T else 0, top_p=0.9, repeat_penalty=p,
                         repeat_window=300), u, hist=hist, label=f"penalty p={p} T={T}")


def test_fused_penalty_paths():
    # windows of <= 256 ids are applied inside the top-K kernel (each
    # workgroup penalises the ids in its own chunk before selecting, and
    # stores them in place); the fast merge, the replay (TopP = 1) and small K
    # all see the penalised row, and the logits equal the reference's in-place
    # result, for penalties above and below 1
    rng = np.random.default_rng(43)
    for V in (20000, 262144):
        B = 6
        L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
        hot = rng.choice(V, 8, replace=False)
        L[:, hot] += np.float32(7.0)
        L[0, 5] = 0.0
        hist = rng.integers(-5, V + 5, (B, 256)).astype(np.int32)
        hist[:, :60] = rng.choice(hot, (B, 60))   # repeats of the largest logits
        hist[:, 60:80] = 5
        hist[1, :] = hot[0]                       # one id 256 times
        hist[2, 100:140] = V - 1                  # the last (short) chunk's last logit
        u = u_stream(rng, B)
        for p in (1.1, 3.0, 0.8):
            for k, tp in ((64, 0.9), (64, 1.0), (5, 0.5)):
                _run(L, dict(temperature=1.0, top_k=k, top_p=tp, repeat_penalty=p,
                             repeat_window=256), u, hist=hist,
                     label=f"fused penalty V={V} p={p} K={k} P={tp}")


def test_fused_penalty_greedy_and_full():
    # windows of <= 256 ids are applied inside the greedy kernel, the full
    # kernel, and (with Min-P) the full path's max pass, in place; logits,
    # tokens and (full path) draws equal the reference's
    rng = np.random.default_rng(47)
    for V in (20000, 262144):
        B = 5
        L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
        hot = rng.choice(V, 8, replace=False)
        L[:, hot] += np.float32(7.0)
        L[0, 5] = 0.0
        hist = rng.integers(-5, V + 5, (B, 200)).astype(np.int32)
        hist[:, :60] = rng.choice(hot, (B, 60))
        hist[:, 60:80] = 5
        hist[1, :] = hot[0]
        hist[2, 100:140] = V - 1
        u = u_stream(rng, B)
        for p in (1.1, 3.0, 0.8, -2.0):
            for kw in (dict(temperature=0.0), dict(temperature=1.0), dict(temperature=0.7, min_p=0.05)):
                _run(L, dict(kw, repeat_penalty=p, repeat_window=200), u, hist=hist,
                     label=f"fused penalty V={V} p={p} {kw}")


# ------------------------------------------------------ stateful sampler ----
def _cfg(s, **kw):
    c = s.DefaultConfig()
    for k, v in kw.items():
        setattr(c, k, v)
    s.SetConfig(c)
    return c


def test_host_process_matches_reference_stream():
    # Process() on host rows with the sampler's own xoshiro256** stream equals
    # the restated reference object call for call (seed 42)
    from vindexllm_amd import TVdxSampler

    rng = np.random.default_rng(3)
    for kw, okw in [(dict(Temperature=1.0, Seed=42), dict(temperature=1.0, seed=42)),
                    (dict(Temperature=0.8, TopK=40, TopP=0.9, Seed=7),
                     dict(temperature=0.8, top_k=40, top_p=0.9, seed=7)),
                    (dict(Temperature=1.0, TopK=3, Seed=42, RepeatPenalty=1.3),
                     dict(temperature=1.0, top_k=3, seed=42, repeat_penalty=1.3))]:
        log(f"[case] stream {kw}")
        ref = O.Sampler()
        ref.set_config(O.make_config(**okw))
        with TVdxSampler(0, 1) as s:
            _cfg(s, **kw)
            for i in range(30):
                L = (rng.standard_normal(3000) * 2).astype(np.float32)
                a, b = L.copy(), L.copy()
                t_gpu = s.Process(a)
                t_ref = ref.process(b)
                assert t_gpu == t_ref, (kw, i)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
                s.AddToHistory(t_gpu)
                ref.add_to_history(t_ref)


def test_host_process_penalty_write_back():
    # the caller's row after Process equals the reference's in-place penalty,
    # bit for bit, with out-of-range, negative and repeated history ids and a
    # window beyond the fused limit (the separate penalty kernel)
    from vindexllm_amd import TVdxSampler

    rng = np.random.default_rng(31)
    V = 5000
    for window, pen in ((8, 2.0), (300, 1.25)):
        log(f"[case] host write-back window={window} RP={pen}")
        ref = O.Sampler()
        ref.set_config(O.make_config(temperature=0.9, top_k=20, seed=5, repeat_penalty=pen,
                                     repeat_window=window))
        with TVdxSampler(0, 1) as s:
            _cfg(s, Temperature=0.9, TopK=20, Seed=5, RepeatPenalty=pen, RepeatWindow=window)
            ids = [-5, V + 3, 7, 7, 0, V - 1] + rng.integers(0, V, window).tolist()
            for t in ids[:window + 2]:
                s.AddToHistory(int(t))
                ref.add_to_history(int(t))
            for i in range(5):
                L = (rng.standard_normal(V) * 3).astype(np.float32)
                L[7], L[0], L[V - 1] = 4.0, -2.5, 0.0
                a, b = L.copy(), L.copy()
                t_gpu, t_ref = s.Process(a), ref.process(b)
                assert t_gpu == t_ref, (window, i)
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (window, i)


def test_ref_invariants_on_gpu():
    # the five sections of testbed/UTest.Sampler.pas, against the GPU sampler
    from vindexllm_amd import TVdxSampler

    log("[case] UTest.Sampler invariants")
    with TVdxSampler() as s:
        c = s.GetConfig()
        assert (c.Temperature, c.TopK, c.TopP, c.MinP, c.RepeatPenalty, c.RepeatWindow, c.Seed) == \
            (0.0, 0, 1.0, 0.0, 1.0, 64, 0)
        _cfg(s, Temperature=0.0)
        L = np.full(10, 0.1, dtype=np.float32)
        L[7] = 5.0
        assert s.Process(L) == 7
        L[7], L[2] = 0.1, 9.9
        assert s.Process(L) == 2
    L = (np.arange(10) * 0.25).astype(np.float32)
    seqs = []
    for _ in range(2):
        with TVdxSampler() as s:
            _cfg(s, Temperature=1.0, Seed=42)
            seqs.append([s.Process(L) for _ in range(50)])
    assert seqs[0] == seqs[1]
    L = np.zeros(10, dtype=np.float32)
    L[[1, 4, 8]] = 10.0
    with TVdxSampler() as s:
        _cfg(s, Temperature=1.0, TopK=3, Seed=42)
        assert all(s.Process(L) in (1, 4, 8) for _ in range(200))
    hits = []
    for rp in (1.0, 2.0):
        with TVdxSampler() as s:
            _cfg(s, Temperature=1.0, RepeatPenalty=rp, Seed=42)
            if rp != 1.0:
                s.AddToHistory(3)
            L1 = np.ones(10, dtype=np.float32)
            hits.append(sum(s.Process(L1.copy()) == 3 for _ in range(200)))
    assert hits[1] < hits[0] and hits[0] > 5


def test_history_ring_semantics():
    from vindexllm_amd import TVdxSampler

    log("[case] history ring")
    with TVdxSampler(0, 3) as s:
        _cfg(s, Temperature=1.0, RepeatWindow=3, Seed=7)
        for t in [10, 11, 12, 13]:
            s.AddToHistory(t, row=1)
        assert s.get_history(1) == ([13, 11, 12], 1)
        assert s.get_history(0) == ([], 0)
        s.ResetHistory(1)
        assert s.get_history(1) == ([], 0)
        _cfg(s, Temperature=1.0, RepeatWindow=4, Seed=7)
        s.AddToHistory(5, row=2)
        assert s.get_history(2) == ([5], 1)
        _cfg(s, Temperature=1.0, RepeatWindow=5, Seed=7)  # window change clears every row
        assert s.get_history(2) == ([], 0)
        import torch
        toks = torch.tensor([1, 2, 3], dtype=torch.int32, device="cuda")
        s.add_to_history_device(toks)
        torch.cuda.synchronize()
        assert [s.get_history(r)[0] for r in range(3)] == [[1], [2], [3]]


def test_rng_streams_per_row():
    # xoshiro: row r draws like a reference sampler with Seed + r; Philox: the
    # uniform of (seed, row, step) restated by the oracle
    import torch
    from vindexllm_amd import VDX_RNG_PHILOX, TVdxSampler

    log("[case] rng per row")
    B, V = 5, 200
    L = np.zeros((B, V), dtype=np.float32)
    with TVdxSampler(0, B) as s:
        _cfg(s, Temperature=1.0, Seed=42)
        d = torch.from_numpy(L).cuda()
        uo = torch.zeros(B, dtype=torch.float32, device="cuda")
        refs = [O.Sampler() for _ in range(B)]
        for r in range(B):
            refs[r].set_config(O.make_config(temperature=1.0, seed=42 + r))
        for step in range(3):
            tok = s.process_device(d, uniforms_out=uo).cpu().numpy()
            got = uo.cpu().numpy()
            for r in range(B):
                assert tok[r] == refs[r].process(L[r].copy())
                assert got[r] == np.float32(int(np.floor(float(got[r]) * 2**24)) / 2**24)
        s.SetRng(VDX_RNG_PHILOX)
        for step in range(3):
            s.process_device(d, uniforms_out=uo)
            got = uo.cpu().numpy()
            for r in range(B):
                assert got[r] == O.philox_uniform(42, r, step)
        s.ResetHistory(-1)  # Seed > 0: reseeds (Philox counters restart)
        s.process_device(d, uniforms_out=uo)
        assert uo.cpu().numpy()[2] == O.philox_uniform(42, 2, 0)


@pytest.mark.parametrize("K,P", [(40, 0.9), (40, 1.0), (100, 0.9), (0, 0.9), (1500, 0.9)])
def test_rng_streams_on_every_path(K, P):
    # the uniform each kernel draws from its row's prefetched state (top-K
    # fast finish, the slot-order kernel, the large-K finish, full softmax,
    # the K > 1024 kernel): xoshiro rows equal reference samplers seeded
    # Seed + r call for call; Philox uniforms equal the (seed, row, step)
    # restatement
    import torch
    from vindexllm_amd import VDX_RNG_PHILOX, TVdxSampler

    log(f"[case] rng streams K={K} P={P}")
    rng = np.random.default_rng(77 + K)
    B, V = 3, 5000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    kw = dict(temperature=1.0, top_k=K, top_p=P)
    with TVdxSampler(0, B) as s:
        _cfg(s, Temperature=1.0, TopK=K, TopP=P, Seed=42)
        d = torch.from_numpy(L).cuda()
        uo = torch.zeros(B, dtype=torch.float32, device="cuda")
        refs = [O.Sampler() for _ in range(B)]
        for r in range(B):
            refs[r].set_config(O.make_config(seed=42 + r, **kw))
        for step in range(3):
            tok = s.process_device(d, uniforms_out=uo).cpu().numpy()
            for r in range(B):
                assert tok[r] == refs[r].process(L[r].copy()), (K, P, step, r)
        s.SetRng(VDX_RNG_PHILOX)
        for step in range(3):
            s.process_device(d, uniforms_out=uo)
            got = uo.cpu().numpy()
            for r in range(B):
                assert got[r] == O.philox_uniform(42, r, step), (K, P, step, r)


def test_injected_u_leaves_rng_untouched():
    import torch
    from vindexllm_amd import TVdxSampler

    B, V = 2, 300
    L = np.zeros((B, V), dtype=np.float32)
    with TVdxSampler(0, B) as s:
        _cfg(s, Temperature=1.0, Seed=9)
        d = torch.from_numpy(L).cuda()
        uo = torch.zeros(B, dtype=torch.float32, device="cuda")
        s.process_device(d, uniforms=torch.tensor([0.5, 0.5], device="cuda"), uniforms_out=uo)
        s.process_device(d, uniforms_out=uo)
        ref = O.Sampler()
        ref.set_config(O.make_config(temperature=1.0, seed=9))
        assert uo.cpu().numpy()[0] == O.lib().vdxo_u24(O.xoshiro_stream(O.seed_state(9), 1)[0])


def test_graph_replay_matches_eager():
    # the sampling call captured in a hipGraph and replayed several times, with
    # eager work in between, gives the eager result every time
    import torch
    from vindexllm_amd import TVdxSampler

    log("[case] graph replay")
    rng = np.random.default_rng(55)
    B, V = 16, 262144
    L, hist = cfg3_inputs(rng, B, V, 256)
    u = torch.from_numpy(u_stream(rng, B)).cuda()
    pristine = torch.from_numpy(L).cuda()
    buf = pristine.clone()
    with TVdxSampler(0, B) as s:
        _cfg(s, Temperature=0.8, TopK=64, TopP=0.95, RepeatPenalty=1.1, RepeatWindow=256, Seed=1)
        for r in range(B):
            s.set_history(r, hist[r])
        tok = torch.zeros(B, dtype=torch.int32, device="cuda")
        eager = s.process_device(buf, uniforms=u).clone()
        eager_logits = buf.clone()
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            s.process_device(buf, uniforms=u, tokens=tok, stream=cs)
        torch.cuda.synchronize()
        for rep in range(4):
            buf.copy_(pristine)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(tok, eager), rep
            assert torch.equal(buf, eager_logits), rep
            _ = (pristine * 2).sum().item()  # unrelated eager work between replays


def test_graph_captured_with_empty_rings_applies_penalty():
    # A decode step [sample, append the token to the ring] captured while every
    # ring is empty, then replayed: from the second replay on the rings hold
    # ids and the penalty must apply, exactly as eager calls apply it.
    import torch
    from vindexllm_amd import TVdxSampler

    log("[case] graph captured with empty rings")
    rng = np.random.default_rng(57)
    B, V = 8, 20000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    for r in range(B):
        L[r, rng.choice(V, 6, replace=False)] += np.float32(6.0)
    u = torch.from_numpy(u_stream(rng, B)).cuda()
    pristine = torch.from_numpy(L).cuda()
    kw = dict(Temperature=1.0, TopK=8, TopP=0.9, RepeatPenalty=3.0, RepeatWindow=16, Seed=3)
    with TVdxSampler(0, B) as s, TVdxSampler(0, B) as ref:
        _cfg(s, **kw)
        _cfg(ref, **kw)
        buf = pristine.clone()
        tok = torch.zeros(B, dtype=torch.int32, device="cuda")
        # one eager call sizes the workspace for V (a call under capture must
        # not allocate); with empty rings and an injected uniform it changes
        # no state
        s.process_device(pristine.clone(), uniforms=u)
        torch.cuda.synchronize()
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            s.process_device(buf, uniforms=u, tokens=tok, stream=cs)
            s.add_to_history_device(tok, stream=cs)
        torch.cuda.synchronize()
        seen_penalty = False
        for step in range(5):
            buf.copy_(pristine)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            rbuf = pristine.clone()
            rtok = ref.process_device(rbuf, uniforms=u)
            ref.add_to_history_device(rtok)
            torch.cuda.synchronize()
            assert torch.equal(tok, rtok), (step, tok, rtok)
            assert torch.equal(buf, rbuf), step
            seen_penalty = seen_penalty or not torch.equal(buf, pristine)
            _ = (pristine * 2).sum().item()  # unrelated eager work between replays
        assert seen_penalty
    log("[done] graph captured with empty rings")
