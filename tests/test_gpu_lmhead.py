"""GPU parity of the Q4_0 lm_head (the reference's shaders/matvec_q4_0.comp,
dispatched from TVdxModel.UnembedToLogits, src/VindexLLM.Model.pas:1258-1270)
and of lm_head + sampling with the logits kept in HBM (Gemma-3-4B tied head:
262144 x 2560 Q4_0, nibbles uniform 0..15, fp16 scales |N(0, 0.02)|, hidden
rows N(0, 1)).

Bar:
  * logits bit-exact against the oracle's restatement of the kernel's
    summation order (oracle/vdx_oracle.c: vdxo_matvec_q4_0_blocked), and within
    the fp32 summation bound of the shader-order restatement;
  * sampling on those logits at the sampler's own bar (tokens, top-K sets and
    order bit-exact, probabilities within 1e-5 relative);
  * end to end against the shader-order logits followed by the oracle
    sampler: the same token except where the two fp32 summation orders can
    flip a decision (a top-K boundary gap or a CDF boundary within the logit
    error), counted and printed.
"""
import os

import numpy as np
import pytest

import npref
from gpu_common import compare, log, oracle_rows, u_stream
from oracle import vdx_oracle as O

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))
U = 2.0 ** -24


def rand_q4_0(rng, rows, in_dim):
    nb = in_dim // 32
    blk = rng.integers(0, 256, (rows, nb, 18), dtype=np.uint8)
    d = np.abs(rng.standard_normal((rows, nb)) * 0.02).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(-1)


def magnitude(w, x, in_dim, rows):
    """sum_e |dequant(W[v][e]) * x[e]| per row (the summation error scale)."""
    W = np.abs(npref.q4_0_dequant(w, in_dim, rows).astype(np.float64))
    return W @ np.abs(x.astype(np.float64))


def gpu_lmhead(w, H, V, D):
    import torch

    from vindexllm_amd import lmhead_q4_0

    dev = torch.device("cuda:0")
    wd = torch.from_numpy(w).to(dev)
    hd = torch.from_numpy(np.ascontiguousarray(H)).to(dev)
    out = lmhead_q4_0(wd, hd, V)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("V,D,B", [(4096 + 77, 256, 1), (4096 + 77, 256, 2), (4096 + 77, 256, 3),
                                   (4096 + 77, 512, 5), (2048, 256, 8), (4096 + 77, 256, 16),
                                   (1000, 256, 17), (1000, 2560, 4), (300, 2560, 1)])
def test_lmhead_logits_bit_exact(V, D, B):
    log(f"[case] lm_head V={V} D={D} B={B}")
    rng = np.random.default_rng(5000 + V + D + B)
    w = rand_q4_0(rng, V, D)
    H = rng.standard_normal((B, D)).astype(np.float32)
    G = gpu_lmhead(w, H, V, D)
    mag = None
    for b in range(B):
        want = O.matvec_q4_0_blocked(w, H[b], D, V)
        assert np.array_equal(G[b].view(np.uint32), want.view(np.uint32)), \
            f"row {b}: {np.flatnonzero(G[b] != want)[:5]}"
        shader = O.matvec_q4_0(w, H[b], D, V).astype(np.float64)
        if mag is None or B > 1:
            mag = magnitude(w, H[b], D, V)
        assert (np.abs(G[b] - shader) <= 2 * (D // 32 + 40) * U * mag).all()
    log(f"[done] lm_head V={V} D={D} B={B}")


def test_lmhead_special_values():
    # zero hidden rows, zero scales, a single non-zero element: exact results
    V, D, B = 512, 256, 3
    rng = np.random.default_rng(77)
    w = rand_q4_0(rng, V, D)
    wb = w.reshape(V, D // 32, 18)
    wb[7, :, 0:2] = 0  # row 7: scale 0 everywhere
    H = np.zeros((B, D), dtype=np.float32)
    H[1, 37] = 1.0
    H[2] = rng.standard_normal(D).astype(np.float32)
    G = gpu_lmhead(w, H, V, D)
    assert (G[0] == 0).all()
    deq = npref.q4_0_dequant(w, D, V)
    assert np.array_equal(G[1], deq[:, 37])
    assert G[2][7] == 0.0
    for b in range(B):
        assert np.array_equal(G[b], O.matvec_q4_0_blocked(w, H[b], D, V))


@pytest.mark.parametrize("packed", [False, True])
def test_lmhead_subnormal_partial_sums(packed):
    # hidden values at and below fp32's smallest normal: the partial sums are
    # subnormal, where the kernel's scaled high-nibble chain (16 s, weights
    # 16 (q - 8)) rounds differently from an unscaled one; the oracle restates
    # the scaled form, so the logits stay bit-exact
    import torch

    from vindexllm_amd import VDX_LMHEAD_PACKED, lmhead, lmhead_pack

    log(f"[case] lm_head subnormal partial sums packed={packed}")
    V, D = 700, 1280
    rng = np.random.default_rng(7100 + packed)
    w = rand_q4_0(rng, V, D)
    H = np.stack([rng.standard_normal(D) * 1e-40,
                  np.where(np.arange(D) % 2 == 0, 1e-37, 1e-41) * rng.standard_normal(D),
                  rng.standard_normal(D)]).astype(np.float32)
    assert (np.abs(H[0]) < np.finfo(np.float32).tiny).all()
    dev = torch.device("cuda:0")
    wd, hd = torch.from_numpy(w).to(dev), torch.from_numpy(H).to(dev)
    wt = O.TENSOR_Q4_0
    if packed:
        wd = lmhead_pack(wd, wt, D, V)
        wt |= VDX_LMHEAD_PACKED
    G = lmhead(wd, wt, hd, V).cpu().numpy()
    for r in range(H.shape[0]):
        want = O.matvec_q4_0_blocked(w, H[r], D, V)
        assert np.array_equal(G[r].view(np.uint32), want.view(np.uint32)), \
            f"row {r}: {np.flatnonzero(G[r].view(np.uint32) != want.view(np.uint32))[:5]}"
    log(f"[done] lm_head subnormal partial sums packed={packed}")


def _cfg5(B, seed):
    rng = np.random.default_rng(seed)
    V, D = 262144, 2560
    w = rand_q4_0(rng, V, D)
    H = rng.standard_normal((B, D)).astype(np.float32)
    u = u_stream(np.random.default_rng(seed + 1000), B)
    return w, H, u, V, D


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("B", [1, 16])
def test_cfg5_lmhead_plus_sampling(B, packed):
    # the config-5 shape (262144 x 2560 Q4_0) in the GGUF layout and in the
    # packed layout the benchmark times: logits bit-exact with the kernel-order
    # restatement either way
    import torch

    from vindexllm_amd import VDX_LMHEAD_PACKED, VDX_TENSOR_Q4_0, TVdxSampler, lmhead_pack

    log(f"[case] C5 lm_head + top-k64/top-p0.95/T1 B={B} packed={packed}")
    w, H, u, V, D = _cfg5(B, 1005 + B)
    cfg = dict(temperature=1.0, top_k=64, top_p=0.95)
    dev = torch.device("cuda:0")
    wd = torch.from_numpy(w).to(dev)
    hd = torch.from_numpy(H).to(dev)
    L = torch.empty(B, V, dtype=torch.float32, device=dev)
    ti = torch.full((B, 64), -1, dtype=torch.int32, device=dev)
    tp = torch.full((B, 64), -1.0, dtype=torch.float32, device=dev)
    fl = torch.zeros(B, dtype=torch.int32, device=dev)
    with TVdxSampler(0, B) as s:
        c = s.DefaultConfig()
        c.Temperature, c.TopK, c.TopP = 1.0, 64, 0.95
        s.SetConfig(c)
        ud = torch.from_numpy(u).to(dev)
        if packed:
            wp = lmhead_pack(wd, VDX_TENSOR_Q4_0, D, V)
            wt = VDX_TENSOR_Q4_0 | VDX_LMHEAD_PACKED
            tok = s.lmhead_device(wp, wt, hd, V, logits=L, uniforms=ud, topk_idx=ti, topk_prob=tp, flags=fl)
            tok2 = s.lmhead_device(wp, wt, hd, V, uniforms=ud)  # the sampler's own workspace
        else:
            tok = s.lmhead_q4_0_device(wd, hd, V, logits=L, uniforms=ud, topk_idx=ti, topk_prob=tp,
                                       flags=fl)
            tok2 = s.lmhead_q4_0_device(wd, hd, V, uniforms=ud)  # the sampler's own workspace
        torch.cuda.synchronize()
    Lg = L.cpu().numpy()
    g = dict(tokens=tok.cpu().numpy(), topk_idx=ti.cpu().numpy(), topk_prob=tp.cpu().numpy(),
             flags=fl.cpu().numpy(), logits_after=Lg)
    assert np.array_equal(g["tokens"], tok2.cpu().numpy())
    # logits: bit-exact with the kernel-order restatement
    for b in range(B):
        want = O.matvec_q4_0_mt(w, H[b], D, V, True, THREADS)
        assert np.array_equal(Lg[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    # sampling on the GPU's logits: the sampler's bar
    orc = oracle_rows(Lg, cfg, u)
    nb = compare(g, orc, cfg, check_logits=False, label=f"C5 B={B}")
    # end to end against the shader's summation order
    flips = 0
    for b in range(B):
        Ls = O.matvec_q4_0_mt(w, H[b], D, V, False, THREADS)
        err = float(np.abs(Ls.astype(np.float64) - Lg[b]).max())
        tok_s, tr_s = O.process_row(Ls.copy(), O.make_config(**cfg), float(u[b]), trace=True)
        if tok_s != g["tokens"][b]:
            srt = np.sort(Ls)[::-1]
            gap = float(srt[63] - srt[64])
            tr_g = orc[b][1]
            bd = min(tr_g.target - tr_g.cdf_lo, tr_g.cdf_hi - tr_g.target) / tr_g.sum_final
            log(f"  row {b}: shader-order token {tok_s} vs {g['tokens'][b]} "
                f"(logit err {err:.2e}, K-boundary gap {gap:.2e}, CDF distance {bd:.2e})")
            assert gap <= 4 * err or bd <= 1e-4, f"row {b}: unexplained token difference"
            flips += 1
    log(f"[done] C5 B={B} packed={packed}: near-boundary draws {nb}, shader-order flips {flips}/{B}, "
        f"flags {sorted(set(g['flags'].tolist()))}")


def test_lmhead_greedy_and_penalty():
    # greedy over lm_head logits is the first index of the maximum; with a
    # repetition penalty the workspace logits are penalised in place first
    import torch

    from vindexllm_amd import TVdxSampler

    V, D, B = 50000, 512, 4
    rng = np.random.default_rng(31)
    w = rand_q4_0(rng, V, D)
    H = rng.standard_normal((B, D)).astype(np.float32)
    hist = rng.integers(0, V, (B, 40)).astype(np.int32)
    dev = torch.device("cuda:0")
    wd = torch.from_numpy(w).to(dev)
    hd = torch.from_numpy(H).to(dev)
    L = torch.empty(B, V, dtype=torch.float32, device=dev)
    with TVdxSampler(0, B) as s:
        c = s.DefaultConfig()
        c.Temperature, c.RepeatPenalty, c.RepeatWindow = 0.0, 1.3, 64
        s.SetConfig(c)
        for r in range(B):
            s.set_history(r, hist[r])
        tok = s.lmhead_q4_0_device(wd, hd, V, logits=L).cpu().numpy()
        torch.cuda.synchronize()
    Lp = L.cpu().numpy()
    for b in range(B):
        raw = O.matvec_q4_0_blocked(w, H[b], D, V)
        pen = npref.penalty(raw, hist[b], 1.3)
        assert np.array_equal(Lp[b].view(np.uint32), pen.view(np.uint32))
        assert tok[b] == int(np.argmax(pen))


# ---- Q8_0 / F16 lm_head and the fused output RMSNorm -----------------------------
def rand_q8_0(rng, rows, in_dim):
    nb = in_dim // 32
    blk = rng.integers(0, 256, (rows, nb, 34), dtype=np.uint8)
    d = np.abs(rng.standard_normal((rows, nb)) * 0.02).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(-1)


def rand_f16(rng, rows, in_dim):
    return (rng.standard_normal((rows, in_dim)) * 0.05).astype(np.float16).view(np.uint8).reshape(-1)


def gpu_lmhead_any(w, wtype, H, V, norm=None, eps=1e-6):
    import torch

    from vindexllm_amd import lmhead

    dev = torch.device("cuda:0")
    wd = torch.from_numpy(w).to(dev)
    hd = torch.from_numpy(np.ascontiguousarray(H)).to(dev)
    nd = torch.from_numpy(norm).to(dev) if norm is not None else None
    out = lmhead(wd, wtype, hd, V, norm_weight=nd, norm_eps=eps)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("wtype", [O.TENSOR_Q8_0, O.TENSOR_F16, O.TENSOR_Q4_0])
@pytest.mark.parametrize("V,D,B,norm", [(4096 + 77, 256, 1, False), (4096 + 77, 256, 3, True),
                                        (2048, 512, 8, False), (1000, 2560, 16, True),
                                        (1000, 2560, 1, True), (300, 256, 17, False),
                                        # in_dim not a whole number of slices (Gemma-3-1B's 1152,
                                        # 45 blocks, one block): the tail blocks
                                        (1000, 1152, 1, False), (777, 1440, 3, True), (300, 32, 2, False)])
def test_lmhead_formats_and_norm_bit_exact(wtype, V, D, B, norm):
    # every format's logits equal the oracle's restatement of the kernel's
    # summation order, on the output-RMSNorm'd rows when the norm is fused
    log(f"[case] lm_head wtype={wtype} V={V} D={D} B={B} norm={norm}")
    rng = np.random.default_rng(7000 + wtype * 100 + V + D + B)
    w = {O.TENSOR_Q8_0: rand_q8_0, O.TENSOR_F16: rand_f16, O.TENSOR_Q4_0: rand_q4_0}[wtype](rng, V, D)
    H = (rng.standard_normal((B, D)) * 4.0).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    G = gpu_lmhead_any(w, wtype, H, V, norm=nw)
    for b in range(B):
        xn = O.rmsnorm(H[b], nw, 1e-6) if norm else H[b]
        want = O.matvec(w, wtype, xn, D, V, True)
        assert np.array_equal(G[b].view(np.uint32), want.view(np.uint32)), \
            f"row {b}: {np.flatnonzero(G[b] != want)[:5]}"
    log(f"[done] lm_head wtype={wtype} V={V} D={D} B={B} norm={norm}")


def test_lmhead_device_q8_0_norm_sampling():
    # UnembedToLogits (norm + Q8_0 head) followed by the sampler, end to end,
    # at Gemma-3-4B's shape with four hidden rows: logits bit-exact with the
    # kernel-order restatement (the shader order's fp32 bound is pinned on the
    # CPU), sampling at the sampler's bar
    import torch

    from vindexllm_amd import VDX_TENSOR_Q8_0, TVdxSampler

    V, D, B = 262144, 2560, 4
    rng = np.random.default_rng(4242)
    w = rand_q8_0(rng, V, D)
    H = (rng.standard_normal((B, D)) * 3.0).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    u = u_stream(np.random.default_rng(4243), B)
    cfg = dict(temperature=1.0, top_k=64, top_p=0.95)
    log("[case] Q8_0 + RMSNorm lm_head + top-k64/top-p0.95 B=4")
    dev = torch.device("cuda:0")
    wd, hd, nd = (torch.from_numpy(a).to(dev) for a in (w, H, nw))
    L = torch.empty(B, V, dtype=torch.float32, device=dev)
    ti = torch.full((B, 64), -1, dtype=torch.int32, device=dev)
    tp = torch.full((B, 64), -1.0, dtype=torch.float32, device=dev)
    fl = torch.zeros(B, dtype=torch.int32, device=dev)
    with TVdxSampler(0, B) as s:
        c = s.DefaultConfig()
        c.Temperature, c.TopK, c.TopP = 1.0, 64, 0.95
        s.SetConfig(c)
        tok = s.lmhead_device(wd, VDX_TENSOR_Q8_0, hd, V, norm_weight=nd, logits=L,
                              uniforms=torch.from_numpy(u).to(dev), topk_idx=ti, topk_prob=tp, flags=fl)
        torch.cuda.synchronize()
    Lg = L.cpu().numpy()
    for b in range(B):
        xn = O.rmsnorm(H[b], nw, 1e-6)
        want = O.matvec(w, O.TENSOR_Q8_0, xn, D, V, True, threads=THREADS)
        assert np.array_equal(Lg[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    g = dict(tokens=tok.cpu().numpy(), topk_idx=ti.cpu().numpy(), topk_prob=tp.cpu().numpy(),
             flags=fl.cpu().numpy(), logits_after=Lg)
    orc = oracle_rows(Lg, cfg, u)
    compare(g, orc, cfg, check_logits=False, label="Q8_0+norm B=4")
    log("[done] Q8_0 + RMSNorm lm_head + sampling")


@pytest.mark.parametrize("wtype", [O.TENSOR_Q4_0, O.TENSOR_Q8_0, O.TENSOR_F16])
def test_lmhead_from_gguf_file(tmp_path, wtype):
    # token_embd.weight and output_norm.weight read from a model file by the
    # library's GGUF reader, copied to the device unchanged, and run through
    # the fused norm + lm_head: bit-exact with the oracle on the same bytes
    import torch

    import ggufw

    from vindexllm_amd import TVdxGGUFReader, lm_head_from_gguf, lmhead

    V, D, B = 4096 + 77, 2560, 3
    log(f"[case] lm_head from GGUF wtype={wtype} V={V} D={D} B={B}")
    rng = np.random.default_rng(9100 + wtype)
    w = {O.TENSOR_Q8_0: rand_q8_0, O.TENSOR_F16: rand_f16, O.TENSOR_Q4_0: rand_q4_0}[wtype](rng, V, D)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    blob, _ = ggufw.build([("general.architecture", ggufw.STR, "gemma3"),
                           ("general.alignment", ggufw.U32, 64)],
                          [("output_norm.weight", [D], 0, nw.tobytes()),
                           ("token_embd.weight", [D, V], wtype, w.tobytes())], alignment=64)
    p = tmp_path / "head.gguf"
    p.write_bytes(blob)
    H = (rng.standard_normal((B, D)) * 3.0).astype(np.float32)
    r = TVdxGGUFReader()
    assert r.Open(str(p)), r.GetErrors()
    dev = torch.device("cuda:0")
    lm = lm_head_from_gguf(r, dev)
    assert (lm["wtype"], lm["in_dim"], lm["vocab"]) == (wtype, D, V)
    out = lmhead(lm["weights"], lm["wtype"], torch.from_numpy(H).to(dev), lm["vocab"],
                 norm_weight=lm["norm_weight"], norm_eps=lm["norm_eps"])
    torch.cuda.synchronize()
    G = out.cpu().numpy()
    for b in range(B):
        want = O.matvec(w, wtype, O.rmsnorm(H[b], nw, 1e-6), D, V, True)
        assert np.array_equal(G[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"[done] lm_head from GGUF wtype={wtype}")


def _pack_ref(w, wtype, D, V):
    """The packed layout restated with numpy: for each 64-row group, slice s
    and piece k, the 64 rows' pieces in row order, then the rows' tail blocks
    (D not a whole number of slices) row after row (rows past V are zero)."""
    bb = {O.TENSOR_Q4_0: 18, O.TENSOR_Q8_0: 34, O.TENSOR_F16: 64}[wtype]
    P, PB, SE = {O.TENSOR_Q4_0: (9, 16, 256), O.TENSOR_Q8_0: (17, 8, 128), O.TENSOR_F16: (8, 16, 64)}[wtype]
    rowbytes = D // 32 * bb
    nw = (V + 63) // 64
    rows = np.zeros((nw * 64, rowbytes), dtype=np.uint8)
    rows[:V] = w.reshape(V, rowbytes)
    ns = D // SE
    mainb = ns * P * PB
    groups = rows.reshape(nw, 64, rowbytes)
    main = groups[:, :, :mainb].reshape(nw, 64, ns, P, PB).transpose(0, 2, 3, 1, 4).reshape(nw, -1)
    tail = groups[:, :, mainb:].reshape(nw, -1)    # each group's rows, their tail bytes in row order
    return np.ascontiguousarray(np.concatenate([main, tail], axis=1)).reshape(-1)


@pytest.mark.parametrize("wtype", [O.TENSOR_Q4_0, O.TENSOR_Q8_0, O.TENSOR_F16])
@pytest.mark.parametrize("D", [512, 1440])
def test_lmhead_pack_layout(wtype, D):
    # the pack kernel's output equals the layout restated with numpy
    import torch

    from vindexllm_amd import lmhead_pack, lmhead_packed_bytes

    V = 200
    log(f"[case] lm_head pack layout wtype={wtype} D={D}")
    rng = np.random.default_rng(9300 + wtype)
    w = {O.TENSOR_Q8_0: rand_q8_0, O.TENSOR_F16: rand_f16, O.TENSOR_Q4_0: rand_q4_0}[wtype](rng, V, D)
    p = lmhead_pack(torch.from_numpy(w).cuda(), wtype, D, V)
    torch.cuda.synchronize()
    want = _pack_ref(w, wtype, D, V)
    assert lmhead_packed_bytes(wtype, D, V) == want.size == p.numel()
    assert np.array_equal(p.cpu().numpy(), want)


@pytest.mark.parametrize("wtype", [O.TENSOR_Q4_0, O.TENSOR_Q8_0, O.TENSOR_F16])
@pytest.mark.parametrize("V,D,B,norm", [(4096 + 77, 256, 1, False), (4096 + 77, 768, 3, True),
                                        (2048, 512, 8, False), (1000, 2560, 16, True),
                                        (300, 2560, 1, True), (63, 256, 17, False),
                                        (1000, 1152, 3, True), (300, 1440, 1, False), (129, 96, 16, False)])
def test_lmhead_packed_matches_gguf_layout(wtype, V, D, B, norm):
    # the packed layout gives the same logits bit for bit (and so the oracle's)
    import torch

    from vindexllm_amd import VDX_LMHEAD_PACKED, lmhead, lmhead_pack

    log(f"[case] packed lm_head wtype={wtype} V={V} D={D} B={B} norm={norm}")
    rng = np.random.default_rng(9400 + wtype * 100 + V + D + B)
    w = {O.TENSOR_Q8_0: rand_q8_0, O.TENSOR_F16: rand_f16, O.TENSOR_Q4_0: rand_q4_0}[wtype](rng, V, D)
    H = (rng.standard_normal((B, D)) * 4.0).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32) if norm else None
    dev = torch.device("cuda:0")
    wd, hd = torch.from_numpy(w).to(dev), torch.from_numpy(H).to(dev)
    nd = torch.from_numpy(nw).to(dev) if norm else None
    wp = lmhead_pack(wd, wtype, D, V)
    a = lmhead(wd, wtype, hd, V, norm_weight=nd)
    b = lmhead(wp, wtype | VDX_LMHEAD_PACKED, hd, V, norm_weight=nd)
    torch.cuda.synchronize()
    G = b.cpu().numpy()
    assert np.array_equal(a.cpu().numpy().view(np.uint32), G.view(np.uint32))
    for r in range(min(B, 3)):
        xn = O.rmsnorm(H[r], nw, 1e-6) if norm else H[r]
        want = O.matvec(w, wtype, xn, D, V, True)
        assert np.array_equal(G[r].view(np.uint32), want.view(np.uint32)), f"row {r}"
    log(f"[done] packed lm_head wtype={wtype} V={V} D={D} B={B}")


def test_lmhead_packed_from_gguf_with_sampling(tmp_path):
    # the head read from a model file, packed on the device, then the fused
    # norm + lm_head + sampling call: the same tokens and logits as the GGUF
    # layout
    import torch

    import ggufw

    from vindexllm_amd import TVdxGGUFReader, TVdxSampler, lm_head_from_gguf

    V, D, B = 8192 + 5, 2560, 4
    log("[case] packed lm_head from GGUF + sampling")
    rng = np.random.default_rng(9500)
    w = rand_q4_0(rng, V, D)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    blob, _ = ggufw.build([], [("output_norm.weight", [D], 0, nw.tobytes()),
                              ("token_embd.weight", [D, V], O.TENSOR_Q4_0, w.tobytes())])
    p = tmp_path / "m.gguf"
    p.write_bytes(blob)
    r = TVdxGGUFReader()
    assert r.Open(str(p))
    dev = torch.device("cuda:0")
    plain = lm_head_from_gguf(r, dev)
    packed = lm_head_from_gguf(r, dev, pack=True)
    H = torch.from_numpy((rng.standard_normal((B, D)) * 3.0).astype(np.float32)).to(dev)
    u = torch.from_numpy(u_stream(rng, B)).to(dev)
    res = []
    for lm in (plain, packed):
        with TVdxSampler(0, B) as s:
            c = s.DefaultConfig()
            c.Temperature, c.TopK, c.TopP = 1.0, 64, 0.95
            s.SetConfig(c)
            L = torch.empty(B, V, device=dev)
            tok = s.lmhead_device(lm["weights"], lm["wtype"], H, V, norm_weight=lm["norm_weight"], logits=L,
                                  uniforms=u)
            torch.cuda.synchronize()
            res.append((tok.cpu().numpy(), L.cpu().numpy()))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1].view(np.uint32), res[1][1].view(np.uint32))
    log("[done] packed lm_head from GGUF + sampling")
