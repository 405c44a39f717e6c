"""GPU parity of the grouped prefill path and of the engine hook (ExpertFfnBatch shape), against
the CPU oracle on arbitrary planes."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import bf16_bits, random_expert_container, rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


@pytest.fixture(scope="module")
def layer(ax, c1_codebook):
    hidden, inter, n = 2048, 1024, 10
    rng = np.random.default_rng(11)
    lay = ax.expert_layout(hidden, inter)
    ex = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n)])
    pool = ax.ExpertPool.from_container(torch.from_numpy(ex.reshape(-1)).cuda(), c1_codebook, hidden, inter)
    torch.cuda.synchronize()
    return ex, pool, hidden, inter


def _oracle(orc, ex, cbf, x, sel, w, hidden, inter):
    y = np.zeros((x.shape[0], hidden), np.float32)
    for t in range(x.shape[0]):
        for j in range(sel.shape[1]):
            e = int(sel[t, j])
            if e < ex.shape[0]:
                orc.expert_ffn(np.ascontiguousarray(ex[e]), cbf, x[t], float(w[t, j]), 10.0, y[t], hidden, inter)
    return y


def _routes(rng, T, k, n, skew=False):
    if skew:   # a Zipf-like head: expert 0 takes most tokens
        p = 1.0 / np.arange(1, n + 1) ** 1.1
        p /= p.sum()
        sel = np.stack([rng.choice(n, k, replace=False, p=p) for _ in range(T)])
    else:
        sel = np.stack([rng.choice(n, k, replace=False) for _ in range(T)])
    return sel.astype(np.uint32), rng.uniform(0.05, 1.0, (T, k)).astype(np.float32)


@pytest.mark.parametrize("T,k,skew,lo", [(9, 6, False, False), (70, 4, True, False), (33, 6, True, True)])
def test_grouped_random_planes(ax, orc, c1_codebook, layer, T, k, skew, lo):
    ex, pool, hidden, inter = layer
    rng = np.random.default_rng(T * 7 + k)
    xf = rng.standard_normal((T, hidden)).astype(np.float32)
    hi = bf16_bits(xf)
    xl = bf16_bits(xf - (hi.astype(np.uint32) << 16).view(np.float32))
    x = (hi.astype(np.uint32) << 16).view(np.float32)
    if lo:
        x = x + (xl.astype(np.uint32) << 16).view(np.float32)
    sel, w = _routes(rng, T, k, ex.shape[0], skew)
    sel[1, 0] = 999  # padding
    gx = torch.from_numpy(hi.view(np.int16)).cuda().view(torch.bfloat16)
    gl = torch.from_numpy(xl.view(np.int16)).cuda().view(torch.bfloat16) if lo else None
    y = ax.expert_ffn_grouped(pool, gx, torch.from_numpy(sel.astype(np.int32)).cuda(),
                              torch.from_numpy(w).cuda(), x_lo=gl)
    torch.cuda.synchronize()
    ref = _oracle(orc, ex, orc.unpack_codebook(c1_codebook), x, sel, w, hidden, inter)
    err = rel_l2(y.cpu().numpy(), ref)
    print(f"T={T} k={k} skew={skew} lo={lo} rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("case", ["single", "one_expert", "one_expert_lo", "every_expert", "all_padding"])
def test_grouped_route_edges(ax, orc, c1_codebook, layer, case):
    """Route shapes at the edges of the grouping: one token with one route; every token on one
    expert (200 tokens: two full wide tiles and a narrow tail with bf16 input, three full tiles
    and a tail with the hi/lo input's 60-token tiles); every token on every expert (k = n); every
    route padding (the output, accumulated into, stays as it was, bit for bit)."""
    ex, pool, hidden, inter = layer
    n = ex.shape[0]
    rng = np.random.default_rng({"single": 1, "one_expert": 2, "one_expert_lo": 3, "every_expert": 4,
                                 "all_padding": 5}[case])
    T, k = {"single": (1, 1), "one_expert": (200, 1), "one_expert_lo": (200, 1), "every_expert": (25, n),
            "all_padding": (5, 2)}[case]
    lo = case == "one_expert_lo"
    xf = rng.standard_normal((T, hidden)).astype(np.float32)
    hi = bf16_bits(xf)
    xl = bf16_bits(xf - (hi.astype(np.uint32) << 16).view(np.float32))
    x = (hi.astype(np.uint32) << 16).view(np.float32)
    if lo:
        x = x + (xl.astype(np.uint32) << 16).view(np.float32)
    w = rng.uniform(0.05, 1.0, (T, k)).astype(np.float32)
    if case == "every_expert":
        sel = np.stack([rng.permutation(n) for _ in range(T)]).astype(np.uint32)
    elif case == "all_padding":
        sel = np.full((T, k), 999, np.uint32)
    else:
        sel = np.full((T, k), 3, np.uint32)
    gx = torch.from_numpy(hi.view(np.int16)).cuda().view(torch.bfloat16)
    gl = torch.from_numpy(xl.view(np.int16)).cuda().view(torch.bfloat16) if lo else None
    y0 = (torch.from_numpy(rng.standard_normal((T, hidden)).astype(np.float32)).cuda() if case == "all_padding"
          else torch.zeros((T, hidden), device="cuda"))
    y = ax.expert_ffn_grouped(pool, gx, torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                              y=y0.clone(), accumulate=True, x_lo=gl)
    torch.cuda.synchronize()
    got = (y - y0).cpu().numpy()
    if case == "all_padding":
        assert torch.equal(y, y0)
        return
    ref = _oracle(orc, ex, orc.unpack_codebook(c1_codebook), x, sel, w, hidden, inter)
    err = rel_l2(got, ref)
    print(f"{case}: T={T} k={k} rel_l2={err:.3e}")
    assert err <= TOL


def test_grouped_is_deterministic(ax, layer):
    ex, pool, hidden, inter = layer
    rng = np.random.default_rng(3)
    T, k = 40, 6
    x = torch.from_numpy(bf16_bits(rng.standard_normal((T, hidden)).astype(np.float32)).view(np.int16)).cuda()
    sel, w = _routes(rng, T, k, ex.shape[0], True)
    args = (pool, x.view(torch.bfloat16), torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda())
    a = ax.expert_ffn_grouped(*args).cpu().numpy()
    b = ax.expert_ffn_grouped(*args).cpu().numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_grouped_batch_invariant(ax, layer):
    """A token's output does not depend on the batch around it: every sum has a fixed order and
    every MFMA column is computed on its own. 3000 tokens (gate/up: 8 row blocks x ~300 tiles =
    thousands of items, so each persistent workgroup runs many of them) against slices of the
    same batch run alone, bit for bit. The slices cover tiles at the start, the middle (an
    expert's tiles split across the slice boundary) and the end."""
    ex, pool, hidden, inter = layer
    rng = np.random.default_rng(5)
    T, k = 3000, 6
    xb = torch.from_numpy(bf16_bits(rng.standard_normal((T, hidden)).astype(np.float32)).view(np.int16)).cuda()
    sel, w = _routes(rng, T, k, ex.shape[0], True)
    sel[7, 2] = 999  # padding
    gs, gw = torch.from_numpy(sel.astype(np.int32)).cuda(), torch.from_numpy(w).cuda()
    full = ax.expert_ffn_grouped(pool, xb.view(torch.bfloat16), gs, gw).cpu().numpy()
    for a, b in ((0, 37), (1400, 1601), (2950, 3000)):
        part = ax.expert_ffn_grouped(pool, xb[a:b].contiguous().view(torch.bfloat16), gs[a:b].contiguous(),
                                     gw[a:b].contiguous()).cpu().numpy()
        np.testing.assert_array_equal(part.view(np.uint32), full[a:b].view(np.uint32), err_msg=f"tokens {a}:{b}")


def test_engine_hook_dim_major_arenas(ax, orc, c1_codebook, layer):
    """affx_expert_ffn_batch with host routes, d_x/d_block f32 [hidden][nb_stride] (accumulated),
    marks every non-padding pair handled and returns their count. One context serves a decode
    batch, a prefill batch, then the decode batch again: the prefill arm must leave the decode's
    persistent counter and flags (at the start of the workspace) zero."""
    from affinity_amd._lib import AffxEngineCtx, lib
    ex, pool, hidden, inter = layer
    k, nbs = 6, 16
    wsb = max(lib().affx_batch_workspace_size(nb, k, pool.n_experts, hidden, inter) for nb in (3, 12))
    ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
    sync_bytes = 256 + 256 * 128
    L = pool.layer()
    for call, nb in enumerate((3, 12, 3)):
        rng = np.random.default_rng(nb + 100 * call)
        x = rng.standard_normal((nb, hidden)).astype(np.float32)
        sel, w = _routes(rng, nb, k, ex.shape[0])
        sel[0, 2] = 4000
        y0 = rng.standard_normal((nb, hidden)).astype(np.float32)
        dx = torch.zeros((hidden, nbs), device="cuda")
        dx[:, :nb] = torch.from_numpy(x.T.copy()).cuda()
        db = torch.zeros((hidden, nbs), device="cuda")
        db[:, :nb] = torch.from_numpy(y0.T.copy()).cuda()
        ctx = AffxEngineCtx(C.pointer(L), 1, dx.data_ptr(), db.data_ptr(), nbs, ws.data_ptr(), wsb,
                            torch.cuda.current_stream().cuda_stream)
        handled = np.zeros(nb * k, np.uint8)
        sel_c = np.ascontiguousarray(sel, np.uint32)
        w_c = np.ascontiguousarray(w, np.float32)
        n = lib().affx_expert_ffn_batch(C.addressof(ctx), 0, sel_c.ctypes.data, w_c.ctypes.data, nb, k,
                                        handled.ctypes.data)
        assert n == nb * k - 1, _lib_err()
        assert handled.reshape(nb, k)[0, 2] == 0 and handled.sum() == n
        got = db.cpu().numpy()
        xr = x
        if nb > 8:  # the grouped arm carries x as a bf16 hi/lo pair
            hi = bf16_bits(x)
            hv = (hi.astype(np.uint32) << 16).view(np.float32)
            xr = hv + (bf16_bits(x - hv).astype(np.uint32) << 16).view(np.float32)
        ref = y0 + _oracle(orc, ex, orc.unpack_codebook(c1_codebook), xr, sel, w, hidden, inter)
        assert rel_l2(got[:, :nb].T, ref) <= TOL, (call, nb)
        np.testing.assert_array_equal(got[:, nb:], 0.0)
        assert int(torch.count_nonzero(ws[:sync_bytes])) == 0, (call, nb)


def _lib_err():
    from affinity_amd._lib import last_error
    return last_error()
