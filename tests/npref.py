"""Independent numpy / pure-Python restatements used to pin the C oracle.

Written separately from oracle/vdx_oracle.c and in a different style
(vectorised numpy where the reference's semantics allow it, explicit
brute force where they do not), so that a slip in one does not repeat in the
other.  Citations are to src/VindexLLM.Sampler.pas in the reference.
"""
from __future__ import annotations

import math

import numpy as np

MASK64 = (1 << 64) - 1


# --- PRNG (Sampler.pas:194-248), Python integers -------------------------
def splitmix64(state: int):
    state = (state + 0x9E3779B97F4A7C15) & MASK64
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return state, z ^ (z >> 31)


def seed(seed_value: int):
    s = seed_value & MASK64
    out = []
    for _ in range(4):
        s, z = splitmix64(s)
        out.append(z)
    return out


def _rotl(x, k):
    return ((x << k) | (x >> (64 - k))) & MASK64


def xoshiro_next(st):
    s0, s1, s2, s3 = st
    result = (_rotl((s1 * 5) & MASK64, 7) * 9) & MASK64
    t = (s1 << 17) & MASK64
    s2 ^= s0
    s3 ^= s1
    s1 ^= s2
    s0 ^= s3
    s2 ^= t
    s3 = _rotl(s3, 45)
    st[:] = [s0, s1, s2, s3]
    return result


def u24(x: int) -> np.float32:
    return np.float32((x >> 40) / 16777216.0)


# --- min-buffer restated as a slot list (Sampler.pas:341-383) --------------
def topk_slots(vals, K):
    """Brute-force restatement of the K-slot min-buffer: returns (slot_values,
    slot_indices, max).  Comparisons are Python float comparisons on float32
    values (NaN compares false, as in the reference)."""
    vals = [np.float32(v) for v in vals]
    M = vals[0]
    slots = []
    for i, v in enumerate(vals):
        if v > M:
            M = v
        if i < K:
            slots.append([v, i])
            continue
        # first slot holding the strict minimum, scanning from slot 0
        m = 0
        for j in range(1, K):
            if slots[j][0] < slots[m][0]:
                m = j
        if v > slots[m][0]:
            slots[m] = [v, i]
    return [s[0] for s in slots], [s[1] for s in slots], M


def topk_tail(slot_vals, slot_idx, M, inv_t, top_p, min_p, u):
    """Softmax / Min-P / Top-P / draw over the slot buffer (:385-459).
    Returns (token, order_idx, order_q, S_final)."""
    v = np.asarray(slot_vals, dtype=np.float32).astype(np.float64)
    q = np.exp((v - np.float64(M)) * np.float64(np.float32(inv_t))).astype(np.float32)
    K = len(q)
    S = 0.0
    for x in q:
        S += float(x)
    if min_p > 0.0:
        best = q[0]
        for x in q[1:]:
            if x > best:
                best = x
        thr = np.float32(best * np.float32(min_p))
        S = 0.0
        for k in range(K):
            if q[k] < thr:
                q[k] = np.float32(0.0)
            else:
                S += float(q[k])
    idx = list(slot_idx)
    if np.float32(top_p) < np.float32(1.0):
        # stable sort, descending by q; equal values keep slot order
        order = sorted(range(K), key=lambda k: (-float(q[k]), k))
        q = q[order]
        idx = [idx[k] for k in order]
        target = float(np.float32(top_p)) * S
        C = 0.0
        S = 0.0
        for k in range(K):
            if C < target and q[k] > 0.0:
                C += float(q[k])
                S += float(q[k])
            else:
                q[k] = np.float32(0.0)
    t = float(np.float32(u)) * S
    C = 0.0
    for k in range(K):
        C += float(q[k])
        if C > t:
            return idx[k], idx, q, S
    return idx[K - 1], idx, q, S


def full_path(L, inv_t, min_p, u):
    """Full-softmax path (:461-527) vectorised: float32 scaling, float64 exp
    rounded to float32, sequential float64 cumsum (np.cumsum is sequential)."""
    s = (np.asarray(L, dtype=np.float32) * np.float32(inv_t)).astype(np.float32)
    # strict '>' running max from s[0]: NaN at s[0] sticks, later NaNs are skipped
    M = s[0] if np.isnan(s[0]) else np.float32(np.nanmax(s))
    q = np.exp(s.astype(np.float64) - np.float64(M)).astype(np.float32)
    if min_p > 0.0:
        thr = np.float32(np.max(q) * np.float32(min_p))
        q = np.where(q < thr, np.float32(0.0), q).astype(np.float32)
    c = np.cumsum(q.astype(np.float64))
    S = c[-1]
    t = float(np.float32(u)) * S
    i = int(np.searchsorted(c, t, side="right"))
    tok = i if i < len(q) else len(q) - 1
    return tok, q, S, t, c


def penalty(L, hist, p):
    """Once-per-occurrence penalty (:285-303), element by element."""
    L = np.array(L, dtype=np.float32, copy=True)
    p = np.float32(p)
    for h in hist:
        if 0 <= h < len(L):
            x = L[h]
            if x > 0:
                L[h] = np.float32(x / p)
            elif x < 0:
                L[h] = np.float32(x * p)
    return L


# --- Q4_0 (shaders/matvec_q4_0.comp:7-15) --------------------------------
def q8_0_dequant(w: np.ndarray, in_dim: int, rows: int) -> np.ndarray:
    """Closed-form dequantisation of rows x in_dim Q8_0 (34-byte blocks: fp16
    d, 32 int8)."""
    nb = in_dim // 32
    blk = w.reshape(rows, nb, 34)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = blk[:, :, 2:34].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(rows, in_dim)


def f16_dequant(w: np.ndarray, in_dim: int, rows: int) -> np.ndarray:
    """rows x in_dim fp16 values, widened."""
    return np.ascontiguousarray(w).view(np.float16).reshape(rows, in_dim).astype(np.float32)


def q4_0_dequant(w: np.ndarray, in_dim: int, rows: int) -> np.ndarray:
    """Closed-form dequantisation of rows x in_dim Q4_0 (18-byte blocks)."""
    nb = in_dim // 32
    blk = w.reshape(rows, nb, 18)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32)  # (rows, nb, 1)
    qs = blk[:, :, 2:18]
    lo = (qs & 0x0F).astype(np.int32) - 8
    hi = (qs >> 4).astype(np.int32) - 8
    vals = np.concatenate([lo, hi], axis=2).astype(np.float32)  # (rows, nb, 32)
    return (vals * d).reshape(rows, in_dim)
