"""The sampler at its largest vocabulary (4 Mi logits = 256 chunks of 16384)
and just beyond it, against the oracle.

At 256 chunks the top-K kernel's chunk quota is 8, so the stored candidates
(>= 2048) can exceed what the general merge holds in LDS, and such rows are
replayed (the reference's min-buffer scan, exact); the full and greedy
kernels reduce 256 chunk records.  Bar: as the other parity tests
(bit-exact tokens, index sets and penalised logits; probabilities within 1e-5
relative).  One logit past the limit the call fails with VDX_E_UNSUPPORTED
and leaves the logits and the token buffer untouched.
"""
import numpy as np
import pytest

from gpu_common import compare, gpu_sample, log, oracle_rows, u_stream
from vindexllm_amd.sampler import VDX_E_UNSUPPORTED, VdxSamplerError

pytestmark = pytest.mark.gpu

VMAX = 256 * 16384  # 4194304


def _logits(rng, B, V):
    L = (3.0 * rng.standard_normal((B, V))).astype(np.float32)
    for r in range(B):
        L[r, rng.choice(V, 16, replace=False)] += np.float32(8.0)
    return L


def _run(L, cfg, u, hist=None, label=""):
    log(f"[case] {label} B={L.shape[0]} V={L.shape[1]} cfg={cfg}")
    g = gpu_sample(L.copy(), cfg, u, hist=hist)
    compare(g, oracle_rows(L, cfg, u, hist=hist), cfg, label=label)
    log(f"[done] {label}: flags {sorted(set(g['flags'].tolist()))}")
    return g


def test_max_vocab_topk():
    rng = np.random.default_rng(81)
    L = _logits(rng, 3, VMAX)
    L[2, VMAX - 1] = 40.0  # the largest logit in the last chunk
    u = u_stream(rng, 3)
    g = _run(L, dict(temperature=1.0, top_k=64, top_p=0.95), u, label="max V top-K")
    assert g["tokens"][2] == VMAX - 1


def test_max_vocab_penalised_topk_minp():
    rng = np.random.default_rng(82)
    B, H = 2, 256
    L = _logits(rng, B, VMAX)
    hist = rng.integers(0, VMAX, (B, H)).astype(np.int32)
    hist[:, :8] = VMAX - 1 - np.arange(8)  # ids in the last chunk
    u = u_stream(rng, B)
    cfg = dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.3, repeat_window=H)
    _run(L, cfg, u, hist=hist, label="max V penalised top-K Min-P")


def test_max_vocab_greedy_and_full():
    rng = np.random.default_rng(83)
    L = _logits(rng, 2, VMAX)
    L[0, VMAX - 3] = L[0, 5] = 60.0  # tie: the lower index wins
    u = u_stream(rng, 2)
    g = _run(L, dict(temperature=0.0), None, label="max V greedy")
    assert g["tokens"][0] == 5
    for minp in (0.0, 0.02):
        _run(L, dict(temperature=0.8, top_k=0, min_p=minp), u, label=f"max V full MinP={minp}")


def test_vocab_beyond_limit_fails():
    import torch

    from vindexllm_amd import TVdxSampler

    V = VMAX + 4
    dev = torch.device("cuda:0")
    x = torch.full((V,), 1.5, dtype=torch.float32, device=dev)
    tok = torch.full((1,), -7, dtype=torch.int32, device=dev)
    with TVdxSampler(0, 1) as s:
        c = s.DefaultConfig()
        c.Temperature, c.TopK, c.TopP = 1.0, 64, 0.95
        s.SetConfig(c)
        log("[case] V = 4 Mi + 4 rejected")
        with pytest.raises(VdxSamplerError) as ei:
            s.process_device(x, tokens=tok, rows=1, vocab=V, row_stride=V)
        assert ei.value.code == VDX_E_UNSUPPORTED
        assert s.GetErrors()
    torch.cuda.synchronize()
    assert int(tok.item()) == -7
    assert bool((x == 1.5).all())
