"""The allocation-free entry point (vdx_sample_device_noalloc) against the
sampler-object entry point (vdx_sampler_process_device) on cuda:0.

Both run the same kernels; the allocation-free one keeps its workspace in the
library's fixed device array, rebuilds each row's state from the caller's
history counts and clears the arrival tickets on every call.  Two calls in a
row (the second on a smaller batch, so stale workspace contents from the
first are present) must give exactly what the sampler object gives for the
same config, rings and injected uniforms: tokens, top-K indices and
probabilities, row flags, consumed uniforms and the penalised logits.
"""
import numpy as np
import pytest

from gpu_common import cfg3_inputs, log, u_stream

pytestmark = pytest.mark.gpu

CASES = [
    # label, rows, vocab, config, history length (0: none)
    ("penalised B=64 V=262144", 64, 262144,
     dict(Temperature=0.8, TopK=64, TopP=0.95, RepeatPenalty=1.1, RepeatWindow=256), 256),
    # Top-P 1: the rows finish in the second (slot-order) kernel on the same workspace
    ("top-p 1 penalised B=16 V=262144", 16, 262144,
     dict(Temperature=0.9, TopK=64, TopP=1.0, RepeatPenalty=1.1, RepeatWindow=64), 64),
    ("top-k 5 / min-p B=8 V=20000", 8, 20000,
     dict(Temperature=1.3, TopK=5, TopP=0.8, MinP=0.05, RepeatPenalty=1.3, RepeatWindow=16), 16),
    ("greedy B=4 V=70001", 4, 70001, dict(Temperature=0.0, RepeatPenalty=1.2, RepeatWindow=32), 20),
    ("full softmax B=3 V=5000 window 300", 3, 5000,
     dict(Temperature=0.7, TopK=0, MinP=0.02, RepeatPenalty=1.5, RepeatWindow=300), 300),
]


def _run_case(label, B, V, kw, H, seed):
    import torch

    from vindexllm_amd import TVdxSampler, sample_device_noalloc

    log(f"[case] noalloc {label}")
    rng = np.random.default_rng(seed)
    if H:
        L, hist = cfg3_inputs(rng, B, V, H)
        counts = rng.integers(H // 2, H + 1, B).astype(np.int32)  # partly filled rings
    else:
        L, hist, counts = (3.0 * rng.standard_normal((B, V))).astype(np.float32), None, None
    u = torch.from_numpy(u_stream(rng, B)).cuda()
    K = max(int(kw.get("TopK", 0)), 1)

    def outputs():
        return (torch.full((B, K), -1, dtype=torch.int32, device="cuda"),
                torch.full((B, K), -1.0, dtype=torch.float32, device="cuda"),
                torch.zeros(B, dtype=torch.int32, device="cuda"),
                torch.zeros(B, dtype=torch.float32, device="cuda"))

    # the sampler object
    a = torch.from_numpy(L).cuda()
    ia, pa, fa, ua = outputs()
    with TVdxSampler(0, B) as s:
        c = s.DefaultConfig()
        for k, v in kw.items():
            setattr(c, k, v)
        s.SetConfig(c)
        if H:
            for r in range(B):
                s.set_history(r, hist[r][:counts[r]])
        ta = s.process_device(a, uniforms=u, topk_idx=ia, topk_prob=pa, flags=fa, uniforms_out=ua)
        torch.cuda.synchronize()
    # the allocation-free entry point
    b = torch.from_numpy(L).cuda()
    ib, pb, fb, ub = outputs()
    hd = torch.from_numpy(hist).cuda() if H else None
    cd = torch.from_numpy(counts).cuda() if H else None
    tb = sample_device_noalloc(c, b, u, history=hd, history_count=cd, topk_idx=ib, topk_prob=pb, flags=fb,
                               uniforms_out=ub)
    torch.cuda.synchronize()
    assert torch.equal(ta, tb), (label, ta, tb)
    assert torch.equal(ia, ib), label
    assert torch.equal(pa, pb), label
    assert torch.equal(fa, fb), label
    assert torch.equal(ua, ub), label
    assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"{label}: penalised logits differ"
    if H:
        assert not torch.equal(b, torch.from_numpy(L).cuda()), f"{label}: no penalty was applied"
    log(f"[done] noalloc {label}")


def test_noalloc_matches_process_device():
    for i, (label, B, V, kw, H) in enumerate(CASES):  # larger first, then smaller batches
        _run_case(label, B, V, kw, H, 9000 + i)


def test_noalloc_rejects_sizes_beyond_the_workspace():
    import torch

    from vindexllm_amd import TVdxSampler, VdxSamplerError, sample_device_noalloc

    c = TVdxSampler.DefaultConfig()
    c.Temperature, c.TopK = 1.0, 64
    # full-size inputs: the calls are refused on the host before any launch
    for B, V in ((257, 262144), (1025, 64)):  # 257 x 16 chunks > 4096; 1025 rows > 1024
        x = torch.zeros((B, V), dtype=torch.float32, device="cuda")
        u = torch.zeros(B, dtype=torch.float32, device="cuda")
        with pytest.raises(VdxSamplerError):
            sample_device_noalloc(c, x, u)
        del x
    torch.cuda.synchronize()
