"""The exact top-K path on cuda:0 against the oracle.

Rows whose draw depends on the reference's min-buffer slot order
(Sampler.pas:341-383, 447-459) -- Top-P = 1 (the draw walks the slots), equal
probabilities at the Top-P cut or the draw, NaN/inf logits -- are finished by
replaying the min-buffer over the logits that can enter it.  Tokens, top-K
sets and the final probabilities must match the oracle at the sampler's bar
(tokens and sets bit-exact, probabilities within 1e-5), on rows built to
stress the replay: every logit entering (ascending rows), none entering after
the fill (descending), integer-valued rows full of ties, NaN at index 0
(nothing ever enters) and elsewhere, +inf and -0/+0.
"""
import time

import numpy as np
import pytest

from gpu_common import cfg1_logits, cfg3_inputs, compare, gpu_sample, log, oracle_rows, u_stream

pytestmark = pytest.mark.gpu

REPLAY = 0x4


def _run(L, cfg, u, hist=None, label="", expect_replay=True):
    g = gpu_sample(L, cfg, u, hist=hist)
    orc = oracle_rows(L, cfg, u, hist=hist)
    compare(g, orc, cfg, label=label)
    if expect_replay:
        assert ((g["flags"] & REPLAY) != 0).all(), (label, g["flags"])
    log(f"[done] {label}")
    return g


@pytest.mark.parametrize("K", [1, 5, 17, 64])
def test_top_p_one_walks_slots(K):
    log(f"[case] top-p 1 K={K}")
    rng = np.random.default_rng(300 + K)
    B, V = 8, 262144
    L = cfg1_logits(rng, B, V)
    u = u_stream(rng, B)
    _run(L, dict(temperature=0.8, top_k=K, top_p=1.0), u, label=f"top-p 1 K={K}")


@pytest.mark.parametrize("V", [261144, 100000, 100003])
def test_top_p_one_ragged_rows(V):
    # a last chunk shorter than the rest (and, at V % 4 != 0, the scalar
    # kernels): the replay re-reads and loads ahead chunks of every length
    log(f"[case] top-p 1 ragged V={V}")
    rng = np.random.default_rng(330 + V % 97)
    B = 4
    L = cfg1_logits(rng, B, V)
    L[1] = np.sort(L[1])  # ascending: every logit enters, every chunk is re-read
    u = u_stream(rng, B)
    for K in (17, 64):
        _run(L, dict(temperature=0.9, top_k=K, top_p=1.0), u, label=f"top-p 1 ragged V={V} K={K}")


def test_top_p_one_penalised_batch():
    log("[case] top-p 1 penalised B=16")
    rng = np.random.default_rng(311)
    L, hist = cfg3_inputs(rng, 16, 262144, 256)
    u = u_stream(rng, 16)
    cfg = dict(temperature=0.8, top_k=64, top_p=1.0, repeat_penalty=1.1, repeat_window=256)
    _run(L, cfg, u, hist=hist, label="top-p 1 penalised")


@pytest.mark.parametrize("P", [1.0, 0.9])
def test_integer_logits_ties(P):
    # integer-valued logits: the K-th value is shared by many logits, so the
    # set itself depends on the slot order
    log(f"[case] integer logits P={P}")
    rng = np.random.default_rng(320)
    B, V = 6, 262144
    L = np.round(3.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[1] = np.round(L[1] / 3.0)  # coarser: fewer distinct values
    u = u_stream(rng, B)
    _run(L, dict(temperature=1.0, top_k=64, top_p=P), u, label=f"integer logits P={P}", expect_replay=False)


def test_every_logit_enters_and_none_enters():
    log("[case] ascending / descending rows")
    V = 65536
    asc = (np.arange(V, dtype=np.float32) * np.float32(1e-3)).astype(np.float32)
    desc = asc[::-1].copy()
    zig = asc.copy()
    zig[1::2] = -zig[1::2]  # every other logit enters
    L = np.stack([asc, desc, zig])
    u = np.array([0.25, 0.5, 0.75], dtype=np.float32)
    for K in (3, 64):
        _run(L, dict(temperature=0.05, top_k=K, top_p=1.0), u, label=f"ascending/descending K={K}")


def test_nan_inf_and_signed_zero_rows():
    log("[case] non-finite rows")
    rng = np.random.default_rng(330)
    B, V = 6, 40000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[0, 0] = np.nan                       # nothing enters: the fill stays
    L[1, 7] = np.nan                       # a NaN slot that is never the minimum
    L[2, 12345] = np.inf                   # +inf enters; M = +inf
    L[3, :64] = np.float32(-0.0)           # -0 and +0 compare equal
    L[3, 64:200] = np.float32(0.0)
    L[4, 20000:20010] = np.nan             # NaN after the fill never enters
    L[5, 3] = np.nan
    L[5, 30000] = np.inf
    u = u_stream(rng, B)
    for P in (1.0, 0.8):
        _run(L, dict(temperature=1.0, top_k=16, top_p=P), u, label=f"non-finite P={P}", expect_replay=False)


def test_nan_slots_in_a_full_buffer():
    # K = 64 with NaN slots in the fill: NaN sorts above +inf and is never the
    # minimum, so each entering logit goes below the NaN entries, up to the
    # highest lane that is not NaN (row 1's ramp: every one of them enters at
    # the top; row 2: one value slot, every entry evicts it)
    log("[case] NaN slots in a full buffer")
    rng = np.random.default_rng(331)
    B, V = 4, 40000
    L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
    L[0, [5, 17, 63]] = np.nan
    L[1, 10:21] = np.nan
    L[1, 64:4000] = np.linspace(-3.0, 9.0, 3936, dtype=np.float32)
    L[2, 1:64] = np.nan
    L[3, 40:64] = np.nan
    L[3, 30000] = np.inf
    u = u_stream(rng, B)
    for P in (1.0, 0.8):
        _run(L, dict(temperature=1.0, top_k=64, top_p=P), u, label=f"NaN slots K=64 P={P}", expect_replay=False)


def test_exact_path_timing_b64():
    # not a bar, a record: the slot-order path on the benchmark's shape
    import torch

    from vindexllm_amd import TVdxSampler

    rng = np.random.default_rng(340)
    B, V = 64, 262144
    L = cfg1_logits(rng, B, V)
    d = torch.from_numpy(L).cuda()
    u = torch.from_numpy(u_stream(rng, B)).cuda()
    fl = torch.zeros(B, dtype=torch.int32, device="cuda")
    with TVdxSampler(0, B) as s:
        c = s.DefaultConfig()
        c.Temperature, c.TopK, c.TopP = 1.0, 64, 1.0
        s.SetConfig(c)
        s.process_device(d, uniforms=u, flags=fl)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            s.process_device(d, uniforms=u)
        torch.cuda.synchronize()
        us = 1e6 * (time.perf_counter() - t0) / 20
    log(f"[record] top-k 64 / top-p 1, B=64 V=262144: {us:.1f} us per call, "
        f"replayed rows {int(((fl.cpu().numpy() & REPLAY) != 0).sum())}")
