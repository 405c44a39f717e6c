"""Helpers shared by the GPU tests (host-side data only; every compute call goes through libaffx)."""
from __future__ import annotations

import numpy as np


def rel_l2(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def bf16_bits(v: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def random_expert_container(rng: np.random.Generator, hidden: int, inter: int, layout,
                            rs_lo: float = 4e-4, rs_hi: float = 2e-3) -> np.ndarray:
    """One expert in container layout with arbitrary planes: random code and field bytes (every
    field value, so every sign/rotation/variant/scale), bf16 row scales in [rs_lo, rs_hi)."""
    stride, off, size = layout
    e = np.zeros(stride, np.uint8)
    rows = (inter, inter, hidden)
    for m in range(3):
        for p in range(2):
            e[off[3 * m + p]:off[3 * m + p] + size[3 * m + p]] = rng.integers(0, 256, size[3 * m + p], dtype=np.uint8)
        rs = bf16_bits(rng.uniform(rs_lo, rs_hi, rows[m]).astype(np.float32))
        e[off[3 * m + 2]:off[3 * m + 2] + size[3 * m + 2]] = rs.view(np.uint8)
    return e


def planes(expert: np.ndarray, layout, which: int):
    """(codes, fields, rscales u16) views of matrix `which` of a container expert."""
    _, off, size = layout
    c = expert[off[3 * which]:off[3 * which] + size[3 * which]]
    f = expert[off[3 * which + 1]:off[3 * which + 1] + size[3 * which + 1]]
    r = expert[off[3 * which + 2]:off[3 * which + 2] + size[3 * which + 2]].view(np.uint16)
    return np.ascontiguousarray(c), np.ascontiguousarray(f), np.ascontiguousarray(r)


def oracle_ffn_tokens(orc, experts: dict, cb_f32, x: np.ndarray, sel: np.ndarray, w: np.ndarray,
                      tokens, hidden: int, inter: int, limit: float = 10.0) -> np.ndarray:
    """The CPU oracle on the given tokens: y[i] = sum_j w[t][j] FFN_{sel[t][j]}(x[t]) with
    t = tokens[i]. experts: expert id -> container bytes (host); other ids are padding."""
    y = np.zeros((len(tokens), hidden), np.float32)
    for i, t in enumerate(tokens):
        for j in range(sel.shape[1]):
            e = int(sel[t, j])
            if e in experts:
                orc.expert_ffn(experts[e], cb_f32, np.ascontiguousarray(x[t], np.float32), float(w[t, j]),
                               limit, y[i], hidden, inter)
    return y


def slot_list(sel: np.ndarray, w: np.ndarray, n_experts: int):
    """The slot list the grouped routes entry builds (the shape of the reference engine's device
    plan, src/gpu/moe_plan.h:144-170): slots sorted by expert and, within an expert, by token;
    expert e owns slots [start[e], start[e+1]); a token's slots in ord[run[t]:run[t+1]] in route
    order. Returns (start, tok, wt, ord, run) as numpy arrays."""
    T, k = sel.shape
    flat = sel.reshape(-1).astype(np.int64)
    valid = (flat >= 0) & (flat < n_experts)
    pairs = np.nonzero(valid)[0]
    order = pairs[np.argsort(flat[pairs], kind="stable")]
    slot_of = np.full(T * k, -1, np.int64)
    slot_of[order] = np.arange(order.size)
    start = np.searchsorted(flat[order], np.arange(n_experts + 1)).astype(np.uint32)
    tok = (order // k).astype(np.uint32)
    wt = w.reshape(-1)[order].astype(np.float32)
    ordv = slot_of[pairs].astype(np.uint32)
    run = np.concatenate([[0], np.cumsum(valid.reshape(T, k).sum(1))]).astype(np.uint32)
    return start, tok, wt, ordv, run
