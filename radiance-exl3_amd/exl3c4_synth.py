"""exl3c4_synth.py -- seeded synthetic workloads for the EXL3 routed-expert path (host side, numpy).

What the reference leaves to its engine and its fixtures, restated for a standalone harness:
  * random experts: uniform random codes (every symbol sequence is a valid trellis, common/exl3_decode.h:31-33),
    f16 sign/scale vectors;
  * the router: softmax over all logits, top_k, optional renormalisation (include/exl3_abi.h:96-98);
  * moe_scatter: a STABLE counting sort of the flat (token, slot) index by expert, dropped slots -1 at the tail
    (include/exl3_abi.h:109-123);
  * Zipf-skewed prefill routing: expert popularity ~ rank^-s over a seeded permutation, each token's top_k distinct
    experts drawn by Gumbel-top-k over log-popularity;
  * the gather: out[t] = sum over ascending slots of expert_w[t, slot] * y[row(t, slot)] in fp32, cast to fp16.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 20261011


def rng_for(cfg: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + cfg + 1000 * salt)


def row_bytes(cols: int, bits: int) -> int:
    return (cols * bits + 7) // 8


def random_codes(rng, rows: int, cols: int, bits: int, entries: int | None = None) -> np.ndarray:
    """Canonical uK planes, uniform random bits: [rows][row_bytes] or [entries][rows][row_bytes]."""
    shape = (rows, row_bytes(cols, bits)) if entries is None else (entries, rows, row_bytes(cols, bits))
    return rng.integers(0, 256, size=shape, dtype=np.uint8)


def sign_scales(rng, n: int, mag: float, entries: int | None = None) -> np.ndarray:
    shape = (n,) if entries is None else (entries, n)
    s = rng.integers(0, 2, size=shape) * 2 - 1
    return (s * mag).astype(np.float16)


def varied_scales(rng, n: int, mag: float, entries: int | None = None) -> np.ndarray:
    """Random signs times magnitudes in [0.5, 1.5) * mag (the spread real checkpoints carry)."""
    shape = (n,) if entries is None else (entries, n)
    s = rng.integers(0, 2, size=shape) * 2 - 1
    return (s * (0.5 + rng.random(shape)) * mag).astype(np.float16)


def normal_f16(rng, shape) -> np.ndarray:
    return rng.standard_normal(shape).astype(np.float32).astype(np.float16)


def router_topk(logits: np.ndarray, top_k: int, renorm: bool = True):
    """softmax over ALL logits, the top_k (ties to the lower id), optional renormalisation."""
    z = logits.astype(np.float64)
    z = np.exp(z - z.max(axis=1, keepdims=True))
    p = z / z.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    w = np.take_along_axis(p, ids, axis=1)
    if renorm:
        w = w / w.sum(axis=1, keepdims=True)
    return ids, w.astype(np.float32)


def zipf_topk(rng, n_tok: int, n_expert: int, top_k: int, s: float = 1.1):
    """Zipf(s) popularity over a seeded permutation of the experts; per token, Gumbel-top-k (distinct experts)."""
    perm = rng.permutation(n_expert)
    pop = np.empty(n_expert)
    pop[perm] = 1.0 / np.arange(1, n_expert + 1, dtype=np.float64) ** s
    logp = np.log(pop / pop.sum())
    g = rng.gumbel(size=(n_tok, n_expert))
    score = logp[None, :] + g
    ids = np.argsort(-score, axis=1, kind="stable")[:, :top_k].astype(np.int32)
    w = np.exp(np.take_along_axis(score, ids, axis=1))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, w


def moe_scatter(expert_ids: np.ndarray, n_expert: int, expert_base: int = 0):
    """sorted_tok i32 [n_tok * top_k] and expert_offset i32 [n_expert + 1] (include/exl3_abi.h:109-123)."""
    flat = np.asarray(expert_ids, dtype=np.int64).reshape(-1) - expert_base
    keep = (flat >= 0) & (flat < n_expert)
    idx = np.nonzero(keep)[0]
    order = idx[np.argsort(flat[idx], kind="stable")]
    counts = np.bincount(flat[idx], minlength=n_expert)
    off = np.zeros(n_expert + 1, np.int32)
    off[1:] = np.cumsum(counts)
    sorted_tok = np.full(flat.size, -1, np.int32)
    sorted_tok[: order.size] = order
    return sorted_tok, off


def gather(y: np.ndarray, sorted_tok: np.ndarray, expert_w: np.ndarray, n_tok: int, top_k: int) -> np.ndarray:
    """out[t] = sum over ascending slots of w[t, slot] * y[row of (t, slot)], fp32, then fp16. y: f32 [T, H]."""
    row_of = np.full(n_tok * top_k, -1, np.int64)
    live = sorted_tok >= 0
    row_of[sorted_tok[live]] = np.nonzero(live)[0]
    out = np.zeros((n_tok, y.shape[1]), np.float32)
    for slot in range(top_k):
        r = row_of[np.arange(n_tok) * top_k + slot]
        ok = r >= 0
        out[ok] += (expert_w[ok, slot][:, None] * y[r[ok]]).astype(np.float32)
    return out.astype(np.float16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
