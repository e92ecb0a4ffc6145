"""Per-row configs and row checkpoints (vdx_sampler_set_row_config,
vdx_sampler_save_row_state / load_row_state) on cuda:0 against the oracle.

A batch whose rows carry their own configs must give, row for row, what a
reference sampler (Sampler.pas:37-91) with that row's config gives: the same
penalised logits, top-K sets and tokens (at the sampler's bar), and, with
the row's own Seed, the same xoshiro256** stream call after call.  A row
restored from a checkpoint continues exactly as the saved row would have.
"""
import numpy as np
import pytest

from gpu_common import compare, log, u_stream
from oracle import vdx_oracle as O

pytestmark = pytest.mark.gpu

# one config per row: every path, the fused (window <= 256) and the separate
# penalty on each, Min-P on both selecting paths, Top-P = 1 (replay), K >= V
ROWS = [
    dict(temperature=0.0),
    dict(temperature=1.0, top_k=64, top_p=0.95),
    dict(temperature=0.7, top_k=5, min_p=0.1),
    dict(temperature=1.2),
    dict(temperature=1.0, min_p=0.05),
    dict(temperature=1.0, top_k=1 << 30),
    dict(temperature=1.0, top_k=40, top_p=0.9, repeat_penalty=1.3, repeat_window=64),
    dict(temperature=0.9, top_k=64, top_p=0.8, repeat_penalty=0.8, repeat_window=512),
    dict(temperature=0.0, repeat_penalty=1.2, repeat_window=32),
    dict(temperature=1.1, repeat_penalty=1.5, repeat_window=128),
    dict(temperature=1.0, top_k=64, top_p=1.0),
    dict(temperature=1.0, top_k=3, top_p=0.5, repeat_penalty=3.0, repeat_window=256),
    dict(temperature=0.9, min_p=0.02, repeat_penalty=1.25, repeat_window=200),
    dict(temperature=0.0, repeat_penalty=1.4, repeat_window=300),
]
PATHS = [0, 1, 1, 2, 2, 2, 1, 1, 0, 2, 1, 1, 2, 0]


def _set(s, row, kw):
    c = s.DefaultConfig()
    c.Temperature = kw.get("temperature", 0.0)
    c.TopK = kw.get("top_k", 0)
    c.TopP = kw.get("top_p", 1.0)
    c.MinP = kw.get("min_p", 0.0)
    c.RepeatPenalty = kw.get("repeat_penalty", 1.0)
    c.RepeatWindow = kw.get("repeat_window", 64)
    c.Seed = kw.get("seed", 0)
    if row is None:
        s.SetConfig(c)
    else:
        s.SetRowConfig(row, c)
    return c


def _okw(kw):
    return {k: v for k, v in kw.items() if k != "seed"}


@pytest.mark.parametrize("V", [20000, 262144])
def test_mixed_row_configs_match_per_row_reference(V):
    import torch

    from vindexllm_amd import TVdxSampler

    rng = np.random.default_rng(700 + V)
    B = len(ROWS)
    log(f"[case] mixed row configs B={B} V={V}")
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    hot = rng.choice(V, 8, replace=False)
    L[:, hot] += np.float32(6.0)
    u = u_stream(rng, B)
    hist = []
    for kw in ROWS:
        w = kw.get("repeat_window", 64)
        h = rng.integers(0, V, w).astype(np.int32)
        h[: w // 4] = rng.choice(hot, w // 4)
        hist.append(h)
    dev = torch.device("cuda:0")
    with TVdxSampler(0, B) as s:
        _set(s, None, dict(temperature=1.0, top_k=64, top_p=0.95))
        for r, kw in enumerate(ROWS):
            _set(s, r, kw)
            s.set_history(r, hist[r])
            got = s.GetRowConfig(r)
            assert got.RepeatWindow == kw.get("repeat_window", 64)
        d = torch.from_numpy(L.copy()).to(dev)
        ti = torch.full((B, 64), -1, dtype=torch.int32, device=dev)
        tp = torch.full((B, 64), -1.0, dtype=torch.float32, device=dev)
        fl = torch.zeros(B, dtype=torch.int32, device=dev)
        tok = s.process_device(d, uniforms=torch.from_numpy(u).to(dev), topk_idx=ti, topk_prob=tp, flags=fl)
        torch.cuda.synchronize()
        g = dict(tokens=tok.cpu().numpy(), topk_idx=ti.cpu().numpy(), topk_prob=tp.cpu().numpy(),
                 flags=fl.cpu().numpy(), logits_after=d.cpu().numpy())
    orc = []
    for r, kw in enumerate(ROWS):
        row = L[r].copy()
        t, tr = O.process_row(row, O.make_config(**_okw(kw)), float(u[r]), hist=hist[r], trace=True)
        orc.append((t, tr, row))
        assert tr.path == PATHS[r], (r, tr.path)
    nb = compare(g, orc, {}, label=f"mixed rows V={V}")
    log(f"[done] mixed row configs V={V}: near-boundary {nb}/{B}, flags {g['flags'].tolist()}")


def test_row_seeds_follow_reference_streams():
    # rows with their own Seed draw what reference samplers with those configs
    # draw, call after call with the history fed back; rows left on the
    # sampler-wide config keep the Seed + r stream
    import torch

    from vindexllm_amd import TVdxSampler

    log("[case] per-row seeds, 12 steps")
    B, V = 4, 3000
    rng = np.random.default_rng(71)
    own = {0: dict(temperature=1.0, top_k=40, top_p=0.9, seed=42, repeat_penalty=1.3, repeat_window=16),
           2: dict(temperature=0.8, seed=7, repeat_penalty=1.1, repeat_window=300)}
    glob = dict(temperature=1.0, top_k=64, top_p=0.95, seed=100)
    refs = []
    for r in range(B):
        kw = own.get(r, dict(glob, seed=100 + r))
        o = O.Sampler()
        o.set_config(O.make_config(**kw))
        refs.append(o)
    dev = torch.device("cuda:0")
    with TVdxSampler(0, B) as s:
        _set(s, None, glob)
        for r, kw in own.items():
            _set(s, r, kw)
        for step in range(12):
            L = (2.0 * rng.standard_normal((B, V))).astype(np.float32)
            d = torch.from_numpy(L.copy()).to(dev)
            tok = s.process_device(d)
            s.add_to_history_device(tok)
            torch.cuda.synchronize()
            tg = tok.cpu().numpy()
            la = d.cpu().numpy()
            for r in range(B):
                row = L[r].copy()
                t = refs[r].process(row)
                assert tg[r] == t, (step, r, tg[r], t)
                assert np.array_equal(la[r].view(np.uint32), row.view(np.uint32)), (step, r)
                refs[r].add_to_history(t)
        for r in range(B):
            assert s.get_history(r)[0] == refs[r].history()[0], r
    log("[done] per-row seeds")


def test_row_checkpoint_restores_the_stream():
    # save every row after a few calls, run on, restore into a fresh sampler
    # with the rows permuted: the restored rows repeat the tokens exactly
    import torch

    from vindexllm_amd import VDX_RNG_PHILOX, TVdxSampler

    log("[case] row checkpoints")
    B, V = 5, 5000
    rng = np.random.default_rng(72)
    steps = [(2.0 * rng.standard_normal((B, V))).astype(np.float32) for _ in range(14)]
    dev = torch.device("cuda:0")

    def run(s, rows_of, from_step, to_step):
        out = []
        for k in range(from_step, to_step):
            L = steps[k][rows_of]
            d = torch.from_numpy(np.ascontiguousarray(L)).to(dev)
            tok = s.process_device(d)
            s.add_to_history_device(tok)
            torch.cuda.synchronize()
            out.append(tok.cpu().numpy())
        return np.stack(out)

    for kind in (None, VDX_RNG_PHILOX):
        ident = np.arange(B)
        with TVdxSampler(0, B) as s:
            if kind is not None:
                s.SetRng(kind)
            _set(s, None, dict(temperature=1.0, top_k=64, top_p=0.95, seed=5, repeat_penalty=1.2,
                               repeat_window=8))
            _set(s, 1, dict(temperature=0.7, top_k=10, seed=9, repeat_penalty=1.4, repeat_window=300))
            _set(s, 3, dict(temperature=1.3, min_p=0.02, seed=11, repeat_penalty=1.1, repeat_window=4))
            run(s, ident, 0, 6)
            blobs = s.save_state()
            want = run(s, ident, 6, 10)
            # ResetHistory reseeds every row with Seed > 0 (Sampler.pas:541-549):
            # a restored row must restart the stream it was taken from, for
            # both generators (the Philox key and counter row included)
            s.ResetHistory(-1)
            want = np.concatenate([want, run(s, ident, 10, 14)])
            cfg1 = s.GetRowConfig(1)
        perm = np.array([3, 0, 4, 1, 2])  # new row j holds saved row perm[j]
        with TVdxSampler(0, B + 2) as s2:
            if kind is not None:
                s2.SetRng(kind)
            for j in range(B):
                s2.load_row_state(j, blobs[perm[j]])
            assert s2.GetRowConfig(3).TopK == cfg1.TopK and s2.GetRowConfig(3).Seed == 9
            got = run(s2, perm, 6, 10)
            s2.ResetHistory(-1)
            got = np.concatenate([got, run(s2, perm, 10, 14)])
        assert np.array_equal(got, want[:, perm]), (kind, got, want[:, perm])
        log(f"[done] row checkpoints kind={kind}")


def test_set_config_takes_every_row_back():
    # SetConfig after per-row configs: every row uses the sampler-wide config;
    # a row with its own seed restarts as row r of Seed + r, rows whose window
    # differed lose their history, the others keep it
    import torch

    from vindexllm_amd import TVdxSampler

    log("[case] set_config after row configs")
    B, V = 3, 1000
    with TVdxSampler(0, B) as s:
        _set(s, None, dict(temperature=1.0, seed=21, repeat_window=8))
        _set(s, 1, dict(temperature=1.0, seed=99, repeat_window=16))
        for r in range(B):
            s.set_history(r, [r + 1, r + 2])
        _set(s, None, dict(temperature=1.0, seed=21, repeat_window=8))
        assert [s.get_history(r)[0] for r in range(B)] == [[1, 2], [], [3, 4]]
        assert s.GetRowConfig(1).Seed == 21
        L = np.zeros((B, V), dtype=np.float32)
        uo = torch.zeros(B, dtype=torch.float32, device="cuda")
        s.process_device(torch.from_numpy(L).cuda(), uniforms_out=uo)
        first = [O.lib().vdxo_u24(O.xoshiro_stream(O.seed_state(21 + r), 1)[0]) for r in range(B)]
        assert uo.cpu().numpy()[1] == np.float32(first[1])
    log("[done] set_config after row configs")


def test_set_config_same_window_keeps_history():
    # After per-row configs widened the ring stride, a SetConfig that changes
    # only the temperature keeps every row's history: the reference clears it
    # only when RepeatWindow changes (Sampler.pas:137-142).
    from vindexllm_amd import TVdxSampler

    log("[case] set_config with an unchanged window")
    with TVdxSampler(0, 2) as s:
        _set(s, None, dict(temperature=1.0, seed=4, repeat_window=8))
        _set(s, 1, dict(temperature=1.0, seed=4, repeat_window=16))
        _set(s, None, dict(temperature=1.0, seed=4, repeat_window=8))
        for r in range(2):
            for t in (r + 5, r + 6, r + 7):
                s.AddToHistory(t, row=r)
        _set(s, None, dict(temperature=0.6, seed=4, repeat_window=8))
        assert [s.get_history(r)[0] for r in range(2)] == [[5, 6, 7], [6, 7, 8]]
        _set(s, None, dict(temperature=0.6, seed=4, repeat_window=9))  # a new window clears
        assert [s.get_history(r)[0] for r in range(2)] == [[], []]
    log("[done] set_config with an unchanged window")


def test_load_row_state_rejects_bad_blobs():
    from vindexllm_amd import VDX_RNG_PHILOX, TVdxSampler, VdxSamplerError

    with TVdxSampler(0, 2) as s:
        _set(s, None, dict(temperature=1.0, seed=3))
        blob = s.save_row_state(0)
        assert len(blob) == 120 + 4 * 64
        # truncated, wrong magic, a window that disagrees with the config
        for bad in (blob[:-4], b"XXXX" + blob[4:], blob[:112] + b"\x05" + blob[113:]):
            with pytest.raises(VdxSamplerError):
                s.load_row_state(1, bad)
        with TVdxSampler(0, 1) as p:
            p.SetRng(VDX_RNG_PHILOX)
            with pytest.raises(VdxSamplerError):
                p.load_row_state(0, blob)
        s.load_row_state(1, blob)
        b2 = s.save_row_state(1)  # the same blob, except that the row now owns its seed
        assert b2[:44] == blob[:44] and b2[48:] == blob[48:] and b2[44] == 1 and blob[44] == 0


def test_mixed_rows_graph_replay_matches_eager():
    # a mixed-path call (greedy, top-K and full rows run side by side on
    # forked streams) captured in a hipGraph and replayed with eager work in
    # between gives the eager result every time
    import torch

    from vindexllm_amd import TVdxSampler

    log("[case] mixed rows graph replay")
    rng = np.random.default_rng(74)
    B, V = len(ROWS), 65536
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    u = torch.from_numpy(u_stream(rng, B)).cuda()
    pristine = torch.from_numpy(L).cuda()
    buf = pristine.clone()
    with TVdxSampler(0, B) as s:
        for r, kw in enumerate(ROWS):
            _set(s, r, kw)
            w = kw.get("repeat_window", 64)
            s.set_history(r, rng.integers(0, V, w).astype(np.int32))
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
            _ = (pristine * 2).sum().item()
    log("[done] mixed rows graph replay")


def test_row_configs_through_the_lmhead_call():
    # the fused norm + packed Q8_0 lm_head + sampling call with per-row
    # configs: each row's token, top-K and logits as the oracle gives them for
    # that row's config on the kernel-order logits
    import torch

    from test_gpu_lmhead import rand_q8_0
    from vindexllm_amd import VDX_LMHEAD_PACKED, VDX_TENSOR_Q8_0, TVdxSampler, lmhead_pack

    V, D = 16384 + 40, 2560
    rows = [ROWS[1], ROWS[0], ROWS[3], ROWS[6], ROWS[2], ROWS[7]]
    B = len(rows)
    log(f"[case] per-row configs through lm_head, B={B}")
    rng = np.random.default_rng(75)
    w = rand_q8_0(rng, V, D)
    H = (rng.standard_normal((B, D)) * 3.0).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    u = u_stream(rng, B)
    hist = [rng.integers(0, V, kw.get("repeat_window", 64)).astype(np.int32) for kw in rows]
    dev = torch.device("cuda:0")
    wp = lmhead_pack(torch.from_numpy(w).to(dev), VDX_TENSOR_Q8_0, D, V)
    L = torch.empty(B, V, device=dev)
    ti = torch.full((B, 64), -1, dtype=torch.int32, device=dev)
    tp = torch.full((B, 64), -1.0, dtype=torch.float32, device=dev)
    fl = torch.zeros(B, dtype=torch.int32, device=dev)
    with TVdxSampler(0, B) as s:
        for r, kw in enumerate(rows):
            _set(s, r, kw)
            s.set_history(r, hist[r])
        tok = s.lmhead_device(wp, VDX_TENSOR_Q8_0 | VDX_LMHEAD_PACKED, torch.from_numpy(H).to(dev), V,
                              norm_weight=torch.from_numpy(nw).to(dev), logits=L, uniforms=torch.from_numpy(u).to(dev),
                              topk_idx=ti, topk_prob=tp, flags=fl)
        torch.cuda.synchronize()
    g = dict(tokens=tok.cpu().numpy(), topk_idx=ti.cpu().numpy(), topk_prob=tp.cpu().numpy(),
             flags=fl.cpu().numpy(), logits_after=L.cpu().numpy())
    orc = []
    for r, kw in enumerate(rows):
        row = O.matvec(w, O.TENSOR_Q8_0, O.rmsnorm(H[r], nw, 1e-6), D, V, True)
        t, tr = O.process_row(row, O.make_config(**_okw(kw)), float(u[r]), hist=hist[r], trace=True)
        orc.append((t, tr, row))
    nb = compare(g, orc, {}, label="rows through lm_head")
    log(f"[done] per-row configs through lm_head: near-boundary {nb}/{B}")


def test_host_process_on_a_row_config():
    # Process (host row 0) with row 0 given its own config: the reference
    # object's stream with that config, logits penalised in place
    from vindexllm_amd import TVdxSampler

    log("[case] host Process with a row config")
    rng = np.random.default_rng(76)
    kw = dict(temperature=0.9, top_k=20, top_p=0.9, repeat_penalty=1.3, repeat_window=8, seed=77)
    ref = O.Sampler()
    ref.set_config(O.make_config(**kw))
    with TVdxSampler(0, 2) as s:
        _set(s, None, dict(temperature=1.0, seed=5))
        _set(s, 0, kw)
        for i in range(20):
            L = (rng.standard_normal(5000) * 2).astype(np.float32)
            a, b = L.copy(), L.copy()
            t_gpu = s.Process(a)
            t_ref = ref.process(b)
            assert t_gpu == t_ref, i
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
            s.AddToHistory(t_gpu)
            ref.add_to_history(t_ref)
    log("[done] host Process with a row config")
