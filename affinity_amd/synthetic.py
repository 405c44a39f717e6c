"""Synthetic inputs of the benchmark configurations (seeded), built on the device by libaffx.

The weights are the reference's own generator (splitmix64 + Box-Muller, bf16-rounded:
src/quant/blockquant.cpp:37-42, 862-869) quantised by the library's GPU quantiser, which is
byte-identical to the reference's quantize_matrix (src/quant/blockquant.cpp:586-791), against
the config-1 codebook the reference fitted (tests/golden/c1_codebook.bin). Seeds:
  S_W = 1000  weights: expert e of a layer from seeds S_W + 3e + {0, 1, 2} (gate, up, down)
  S_X = 7     activations
  S_R = 11    router logits (+ layer)
  S_Z = 13    Zipf expert permutation and sampling (prefill)
"""
from __future__ import annotations

import os
import time

import numpy as np

S_W, S_X, S_R, S_Z = 1000, 7, 11, 13
H, I, E, K = 4096, 2048, 256, 6
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CODEBOOK = os.path.join(ROOT, "tests", "golden", "c1_codebook.bin")


def c1_codebook() -> np.ndarray:
    """The config-1 codebook (uint32[2048] packed E4M3 quads) the reference fitted."""
    return np.fromfile(CODEBOOK, dtype="<u4")


def softmax_topk(logits, k: int = K):
    """Top-k by logit (ties -> lower id), weights = softmax renormalised over the k, computed in
    double: the configs' routing rule. logits: torch tensor [..., n]."""
    import torch
    order = torch.sort(logits, dim=-1, descending=True, stable=True).indices[..., :k]
    top = torch.gather(logits, -1, order).double()
    w = torch.softmax(top, dim=-1).float()
    return order.to(torch.int32).contiguous(), w.contiguous()


def zipf_routes(T: int, n: int = E, k: int = K, s: float = 1.1, seed: int = S_Z):
    """Config-4 routes: 6 distinct experts per token drawn with Zipf(s) popularity over a seeded
    permutation of the experts; weights = softmax of per-token N(0,1) logits over the 6."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n)
    p = 1.0 / np.arange(1, n + 1) ** s
    p /= p.sum()
    sel = np.empty((T, k), np.int32)
    for t in range(T):
        sel[t] = perm[rng.choice(n, k, replace=False, p=p)]
    lg = rng.standard_normal((T, k))
    w = np.exp(lg - lg.max(1, keepdims=True))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return sel, w


def build_layer_container(ax, torch, n: int = E, hidden: int = H, inter: int = I, log=None):
    """The config-2 layer in container layout, on the device: uint8 [n * stride]."""
    cbf = torch.from_numpy(ax.codebook_floats(c1_codebook())).cuda()
    stride = ax.expert_layout(hidden, inter)[0]
    cont = torch.empty(n * stride, dtype=torch.uint8, device="cuda")
    t0 = time.time()
    for e0 in range(0, n, 32):
        cnt = min(32, n - e0)
        ax.fill_synthetic_experts(cont, e0, cnt, cbf, lambda e: S_W + 3 * e, hidden, inter)
        torch.cuda.synchronize()
        if log:
            log(f"quantised experts {e0 + cnt}/{n} ({time.time() - t0:.1f} s)")
    return cont


def expert_bytes(cont, e: int, stride: int) -> np.ndarray:
    """Expert e of a device container as a host uint8 array."""
    return cont[e * stride:(e + 1) * stride].cpu().numpy()


def prefill_sample(sel: np.ndarray, n_experts: int, n: int = 64, tiles=(96, 60), seed: int = 5):
    """A deterministic subsample of prefill tokens that covers the tiling: tokens in the first,
    middle and last tile (and at every tile edge) of the most popular expert, the single token
    of every 1-token tail tile, then seeded random tokens up to n. The grouped path gives each
    expert's tokens consecutive slots in token order and cuts them into tiles of `tiles` tokens
    (96 gate/up with a bf16 input, 60 down and with a hi/lo input)."""
    T, k = sel.shape
    flat = sel.reshape(-1)
    toks = {e: [] for e in range(n_experts)}
    for i, e in enumerate(flat):
        if 0 <= e < n_experts:
            toks[int(e)].append(i // k)
    pick: list[int] = []

    def add(t):
        if t not in pick and len(pick) < n:
            pick.append(int(t))

    head = max(toks, key=lambda e: len(toks[e]))
    ht = toks[head]
    for tt in tiles:
        nt = (len(ht) + tt - 1) // tt
        for j in (0, nt // 2, nt - 1):
            for pos in (j * tt, min(len(ht), (j + 1) * tt) - 1):
                add(ht[pos])
    for tt in tiles:
        for e in range(n_experts):
            if len(toks[e]) % tt == 1:
                add(toks[e][-1])
    rng = np.random.default_rng(seed)
    for t in rng.permutation(T):
        add(t)
    return np.array(sorted(pick[:n]), np.int64), head, len(ht)

