"""GPU parity of the decode path: layout, dequant (bit-exact), fp8-MFMA decode FFN (rel-L2).

Every compute call goes through libaffx.so's C-ABI; the CPU oracle (oracle/liboracle.so) is the
checker. Arbitrary planes (random code and field bytes) exercise every field value; the
quantised synthetic experts of the benchmark configs come from the GPU quantiser, whose bytes
test_gpu_quant.py pins to the reference's golden hashes.
"""
import ctypes as C
import os

import numpy as np
import pytest

from gpu_util import planes, random_expert_container, rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-3  # expert outputs: relative L2 vs the CPU path (fp32 accumulate)


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def _pool_from_numpy(ax, experts: np.ndarray, cb_packed, hidden, inter):
    t = torch.from_numpy(experts.reshape(-1)).cuda()
    pool = ax.ExpertPool.from_container(t, cb_packed, hidden, inter)
    torch.cuda.synchronize()
    return pool


def _mfma(lib, a, b):
    ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    d = torch.zeros(64 * 4, dtype=torch.float32, device="cuda")
    assert lib().affx_selftest_mfma_fp8(ga.data_ptr(), gb.data_ptr(), d.data_ptr(), 0) == 0
    torch.cuda.synchronize()
    d = d.cpu().numpy().reshape(64, 4)
    got = np.zeros((16, 16))
    for l in range(64):
        for v in range(4):
            got[4 * (l // 16) + v, l % 16] = d[l, v]
    return got


def _lane_product(tbl, a, b):
    av, bv = tbl[a].astype(np.float64), tbl[b].astype(np.float64)
    ref = np.zeros((16, 16))
    for i in range(16):
        for j in range(16):
            ref[i, j] = sum(np.dot(av[i + 16 * g], bv[j + 16 * g]) for g in range(4))
    return ref


def test_mfma_fp8_lane_layout(ax):
    """A/B lane l = (row/col l%16, k-group l/16) with the same k order; D lane l elem v =
    D[4*(l/16)+v][l%16]; bytes read as OCP E4M3 (bias 7)."""
    from affinity_amd._lib import lib
    rng = np.random.default_rng(1)
    tbl = ax.e4m3_table()
    # exact case: entries +-{0.5, 1, 2, 4} (E4M3 0x30/0x38/0x40/0x48 and negatives) give integer
    # multiples of 1/4 whose sums are exact in any accumulator
    pick = np.array([0x30, 0x38, 0x40, 0x48, 0xB0, 0xB8, 0xC0, 0xC8], np.uint8)
    a = pick[rng.integers(0, 8, (64, 32))]
    b = pick[rng.integers(0, 8, (64, 32))]
    np.testing.assert_array_equal(_mfma(lib, a, b), _lane_product(tbl, a, b))
    # whole range (no NaN encodings): the accumulation is not IEEE-exact over 2^-9..448 products,
    # so check the layout to a loose relative tolerance
    def rand_bytes():
        x = rng.integers(0, 256, (64, 32), dtype=np.uint8)
        x[(x & 0x7F) == 0x7F] ^= 1
        return x
    a, b = rand_bytes(), rand_bytes()
    ref = _lane_product(tbl, a, b)
    got = _mfma(lib, a, b)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-3


def test_mfma_fp8_accumulation_window(ax):
    """How the fp8 MFMA sums its 128 products (the numerics the kernels rely on): exact within 13
    bits of the largest product of a group of 8; a product 14 bits below it in the same group is
    dropped; products in other groups are kept; on random codes over the whole E4M3 range, the
    error of one MFMA stays below 2^-10 of its largest product."""
    from affinity_amd._lib import lib
    tbl = ax.e4m3_table().astype(np.float64)
    enc = {v: int(np.flatnonzero(tbl[:0x7F] == v)[0]) for v in (1.0, 16.0, 256.0, 2.0 ** -6, 2.0 ** -8, 2.0 ** -9)}

    def row0(big, small, n, bsmall=1.0):
        # A row 0 and B column 0 live in lanes 0, 16, 32, 48 (32 k values each), k-major
        a = np.zeros((64, 32), np.uint8)
        b = np.zeros((64, 32), np.uint8)
        a[0, 0], b[0, 0] = enc[big], enc[1.0]
        for k in range(1, 1 + n):
            a[16 * (k // 32), k % 32], b[16 * (k // 32), k % 32] = enc[small], enc[bsmall]
        return _mfma(lib, a, b)[0, 0], _lane_product(tbl, a, b)[0, 0]

    got, ref = row0(16.0, 2.0 ** -9, 127)          # 2^-13 of the largest: kept
    assert got == ref == 16.0 + 127 * 2.0 ** -9
    got, ref = row0(1.0, 2.0 ** -6, 1, 2.0 ** -8)   # 2^-14 of the largest, same group: dropped
    assert ref == 1.0 + 2.0 ** -14 and got == 1.0
    got, ref = row0(256.0, 2.0 ** -6, 127)         # 2^-14: only the 7 in the large one's group are lost
    assert ref - got == 7 * 2.0 ** -6
    rng = np.random.default_rng(5)
    worst = 0.0
    for _ in range(10):
        a = rng.integers(0, 256, (64, 32), dtype=np.uint8)
        b = rng.integers(0, 256, (64, 32), dtype=np.uint8)
        a[(a & 0x7F) == 0x7F] ^= 1
        b[(b & 0x7F) == 0x7F] ^= 1
        got, ref = _mfma(lib, a, b), _lane_product(tbl, a, b)
        av, bv = tbl[a], tbl[b]
        pmax = np.array([[max(np.abs(av[i + 16 * g] * bv[j + 16 * g]).max() for g in range(4)) for j in range(16)]
                         for i in range(16)])
        worst = max(worst, float((np.abs(got - ref) / pmax).max()))
    print(f"random E4M3 codes: worst MFMA error {worst:.3e} of the largest product (2^{np.log2(worst):.2f})")
    assert worst < 2.0 ** -10


@pytest.mark.parametrize("hidden,inter", [(1024, 1024), (4096, 2048)])
def test_device_permutation_matches_host(ax, hidden, inter):
    from affinity_amd._lib import lib
    rng = np.random.default_rng(hidden + inter)
    lay = ax.expert_layout(hidden, inter)
    src = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(2)])
    host = np.zeros_like(src)
    for e in range(2):
        assert lib().affx_expert_to_device_layout(src[e].ctypes.data, host[e].ctypes.data, hidden, inter) == 0
    pool = _pool_from_numpy(ax, src, np.full(2048, 0x38383838, np.uint32), hidden, inter)
    dev = pool.data.cpu().numpy().reshape(2, -1)
    _, off, size = lay
    for p in range(9):  # compare planes (padding between planes is not copied)
        np.testing.assert_array_equal(dev[:, off[p]:off[p] + size[p]], host[:, off[p]:off[p] + size[p]])


@pytest.mark.parametrize("hidden,inter", [(1024, 1024), (4096, 2048)])
def test_dequant_bit_exact_random_planes(ax, orc, c1_codebook, hidden, inter):
    rng = np.random.default_rng(7 + hidden)
    lay = ax.expert_layout(hidden, inter)
    ex = random_expert_container(rng, hidden, inter, lay)
    pool = _pool_from_numpy(ax, ex[None], c1_codebook, hidden, inter)
    cbf = orc.unpack_codebook(c1_codebook)
    for which in range(3):
        rows, cols = ((inter, hidden), (inter, hidden), (hidden, inter))[which]
        got = ax.dequant_matrix(pool, 0, which).cpu().numpy()
        ref = orc.dequantize(*planes(ex, lay, which), rows, cols, cbf)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def _oracle_ffn(orc, experts, cbf, x, sel, w, hidden, inter, limit=10.0):
    M = x.shape[0]
    y = np.zeros((M, hidden), np.float32)
    for t in range(M):
        for j in range(sel.shape[1]):
            e = int(sel[t, j])
            if e >= experts.shape[0]:
                continue
            orc.expert_ffn(np.ascontiguousarray(experts[e]), cbf, x[t], float(w[t, j]), limit, y[t],
                           hidden, inter)
    return y


def _run_decode(ax, pool, x, sel, w, **kw):
    gx = torch.from_numpy(x).cuda()
    gs = torch.from_numpy(sel.astype(np.int32)).cuda()
    gw = torch.from_numpy(w.astype(np.float32)).cuda()
    y = ax.expert_ffn_decode(pool, gx, gs, gw, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.fixture(scope="module")
def random_layer(ax, c1_codebook):
    hidden, inter, n = 2048, 1024, 12
    rng = np.random.default_rng(99)
    lay = ax.expert_layout(hidden, inter)
    ex = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n)])
    return ex, _pool_from_numpy(ax, ex, c1_codebook, hidden, inter), hidden, inter


@pytest.mark.parametrize("M,k", [(1, 6), (3, 4), (5, 6), (6, 6), (8, 6), (2, 1), (1, 12), (8, 12), (1, 16), (8, 16)])
def test_decode_random_planes(ax, orc, c1_codebook, random_layer, M, k):
    """Up to the plan's limits: top-k 16 (the reference's limit) and 8 x 16 = 128 routes; k = 16
    exceeds the layer's 12 experts, so those routes repeat experts (each repeat counts again)."""
    ex, pool, hidden, inter = random_layer
    rng = np.random.default_rng(M * 10 + k)
    x = (rng.standard_normal((M, hidden)) * 0.5).astype(np.float32)
    n = ex.shape[0]
    sel = np.stack([rng.choice(n, k, replace=k > n) for _ in range(M)]).astype(np.uint32)
    w = rng.uniform(0.05, 1.0, (M, k)).astype(np.float32)
    got = _run_decode(ax, pool, x, sel, w)
    ref = _oracle_ffn(orc, ex, orc.unpack_codebook(c1_codebook), x, sel, w, hidden, inter)
    err = rel_l2(got, ref)
    print(f"M={M} k={k} rel_l2={err:.3e}")
    assert err <= TOL


def test_decode_padding_duplicates_accumulate_dim_major(ax, orc, c1_codebook, random_layer):
    """Padding ids (>= n_experts) are skipped, a repeated expert counts twice, accumulate adds
    into y, and the dim-major [hidden][nb] arenas of the engine are addressed correctly."""
    ex, pool, hidden, inter = random_layer
    rng = np.random.default_rng(5)
    M, k, n = 4, 6, ex.shape[0]
    x = rng.standard_normal((M, hidden)).astype(np.float32)
    sel = np.stack([rng.choice(n, k, replace=False) for _ in range(M)]).astype(np.uint32)
    sel[0, 5] = n + 3          # padding
    sel[1, 4] = sel[1, 0]      # duplicate
    sel[2, :] = 1000           # a token with nothing routed
    w = rng.uniform(0.1, 1.0, (M, k)).astype(np.float32)
    y0 = rng.standard_normal((M, hidden)).astype(np.float32)
    nb = 8                     # arena stride (nb_stride) larger than M
    xd = np.zeros((hidden, nb), np.float32)
    xd[:, :M] = x.T
    yd = np.zeros((hidden, nb), np.float32)
    yd[:, :M] = y0.T
    gx, gy = torch.from_numpy(xd).cuda(), torch.from_numpy(yd).cuda()
    ax.expert_ffn_decode(pool, gx[:, :M], torch.from_numpy(sel.astype(np.int32)).cuda(),
                         torch.from_numpy(w).cuda(), y=gy[:, :M], accumulate=True, dim_major=True)
    torch.cuda.synchronize()
    got = gy.cpu().numpy()
    ref = y0 + _oracle_ffn(orc, ex, orc.unpack_codebook(c1_codebook), x, sel, w, hidden, inter)
    assert rel_l2(got[:, :M].T, ref) <= TOL
    np.testing.assert_array_equal(got[:, M:], 0.0)      # columns beyond M untouched
    np.testing.assert_array_equal(got[:, 2], y0[2])     # nothing routed: y unchanged


def test_decode_declines(ax, random_layer):
    from affinity_amd._lib import AffxDeclined
    ex, pool, hidden, inter = random_layer
    x = torch.zeros((9, hidden), device="cuda")
    sel = torch.zeros((9, 6), dtype=torch.int32, device="cuda")
    w = torch.zeros((9, 6), device="cuda")
    with pytest.raises(AffxDeclined):
        ax.expert_ffn_decode(pool, x, sel, w)


# ---- the persistent (fused) launch against the staged launches -----------------------------------

def _random_device_pool(ax, c1_codebook, n, hidden, inter, seed):
    """A pool filled on the device with arbitrary planes: random code/field bytes (any byte
    permutation of random bytes is random, so they are written in device layout directly) and
    bf16 row scales in [4e-4, 2e-3)."""
    pool = ax.ExpertPool.empty(n, c1_codebook, hidden, inter)
    g = torch.Generator(device="cuda").manual_seed(seed)
    stride, off, size = ax.expert_layout(hidden, inter)
    raw = pool.data.view(n, stride)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, device="cuda", generator=g))
    for m in range(3):
        o, sz = off[3 * m + 2], size[3 * m + 2]
        rs = 4e-4 + 1.6e-3 * torch.rand((n, sz // 2), device="cuda", generator=g)
        raw[:, o:o + sz] = rs.to(torch.bfloat16).view(torch.uint8)
    torch.cuda.synchronize()
    return pool


@pytest.mark.parametrize("M,k,pick", [(1, 6, 256), (2, 6, 256), (5, 6, 256), (8, 6, 256), (8, 6, 8), (1, 16, 256),
                                      (4, 16, 256)])
def test_fused_decode_identical_to_staged_full_layer(ax, orc, c1_codebook, M, k, pick):
    """The benchmark layer shape (256 experts, hidden 4096, inter 2048): the one-launch decode
    equals the three staged launches bit for bit (same MFMA operands, same summation order),
    leaves its counters zero, and matches the oracle on every token. pick = 8: every route names
    one of 8 experts, so most slots serve six or more tokens and take the fused kernel's second
    pass over their weights. Top-16 routes give more gate/up items than one pass of the grid holds,
    so batch 1 runs the rounds kernel too."""
    hidden, inter, n = 4096, 2048, 256
    pool = _random_device_pool(ax, c1_codebook, n, hidden, inter, seed=17 + M)
    rng = np.random.default_rng(100 + M + pick)
    x = torch.from_numpy((rng.standard_normal((M, hidden)) * 0.7).astype(np.float32)).cuda()
    sel_np = np.stack([rng.choice(pick, k, replace=False) for _ in range(M)]).astype(np.int32)
    sel = torch.from_numpy(sel_np).cuda()
    w = torch.from_numpy(rng.uniform(0.05, 1.0, (M, k)).astype(np.float32)).cuda()
    ws = ax.DecodeWorkspace(M, k, hidden, inter)
    ys = ax.expert_ffn_decode(pool, x, sel, w, staged=True, workspace=ax.DecodeWorkspace(M, k, hidden, inter))
    y1 = ax.expert_ffn_decode(pool, x, sel, w, workspace=ws)
    y2 = ax.expert_ffn_decode(pool, x, sel, w, workspace=ws)   # reuses the counters
    torch.cuda.synchronize()
    assert torch.equal(y1, ys) and torch.equal(y2, ys)
    assert ws.error_flags() == 0
    assert int(ws.buf[:8].view(torch.int32).abs().sum().item()) == 0, "counters not reset"
    # oracle on the routed experts (every token), brought back to container layout
    stride, _, _ = ax.expert_layout(hidden, inter)
    from affinity_amd._lib import lib
    ids = sorted(set(int(e) for e in sel_np.reshape(-1)))
    dev = pool.data.view(n, stride)[torch.tensor(ids, dtype=torch.int64, device="cuda")].cpu().numpy()
    cont = np.zeros_like(dev)
    for j in range(len(ids)):
        assert lib().affx_expert_from_device_layout(dev[j].ctypes.data, cont[j].ctypes.data, hidden, inter) == 0
    remap = np.vectorize({e: j for j, e in enumerate(ids)}.get)(sel_np).astype(np.uint32)
    ref = _oracle_ffn(orc, cont, orc.unpack_codebook(c1_codebook), x.cpu().numpy(), remap, w.cpu().numpy(),
                      hidden, inter)
    err = rel_l2(y1.cpu().numpy(), ref)
    print(f"fused M={M} full layer, {len(ids)} experts: rel_l2={err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("M,nb", [(1, 16), (3, 16), (6, 16), (8, 16), (8, 8), (7, 12), (6, 10)])
def test_fused_decode_dim_major_arena(ax, c1_codebook, M, nb):
    """The engine's dim-major batch arena x[h * nb + t] (16 = the reference's narrow-batch
    stride, src/gpu/batch_kernels.h:57) at the benchmark layer shape: equal bit for bit to the
    token-major call and to the staged launches. The arena's unused token slots hold huge values
    that must not reach the result (the 6-8 token decode reads four tokens of a row at once)."""
    hidden, inter, n, k = 4096, 2048, 256, 6
    pool = _random_device_pool(ax, c1_codebook, n, hidden, inter, seed=31 + M)
    rng = np.random.default_rng(200 + M + nb)
    xn = (rng.standard_normal((M, hidden)) * 0.7).astype(np.float32)
    x = torch.from_numpy(xn).cuda()
    xd = torch.full((hidden, nb), 3e37, device="cuda")
    xd[:, :M] = x.t()
    sel = torch.from_numpy(np.stack([rng.choice(n, k, replace=False) for _ in range(M)]).astype(np.int32)).cuda()
    w = torch.from_numpy(rng.uniform(0.05, 1.0, (M, k)).astype(np.float32)).cuda()
    ws = ax.DecodeWorkspace(M, k, hidden, inter)
    yt = ax.expert_ffn_decode(pool, x, sel, w, workspace=ws)
    ys = ax.expert_ffn_decode(pool, x, sel, w, staged=True, workspace=ax.DecodeWorkspace(M, k, hidden, inter))
    yd = torch.zeros((hidden, nb), device="cuda")
    ax.expert_ffn_decode(pool, xd[:, :M], sel, w, y=yd[:, :M], workspace=ws, dim_major=True)
    torch.cuda.synchronize()
    assert torch.equal(yt, ys)
    assert torch.equal(yd[:, :M].t(), yt)
    assert torch.equal(yd[:, M:], torch.zeros_like(yd[:, M:]))
    assert ws.error_flags() == 0


def test_fused_decode_graph_replays(ax, c1_codebook):
    """Captured in a HIP graph, the persistent decode replays to the eager result every time
    (its counters are reset by the kernel itself, nothing is memset)."""
    hidden, inter, n, k = 4096, 2048, 64, 6
    pool = _random_device_pool(ax, c1_codebook, n, hidden, inter, seed=5)
    rng = np.random.default_rng(6)
    x = torch.from_numpy(rng.standard_normal((1, hidden)).astype(np.float32)).cuda()
    sel = torch.from_numpy(rng.choice(n, k, replace=False).astype(np.int32)[None, :]).cuda()
    w = torch.from_numpy(rng.uniform(0.1, 1.0, (1, k)).astype(np.float32)).cuda()
    ws = ax.DecodeWorkspace(1, k, hidden, inter)
    y = torch.zeros((1, hidden), device="cuda")
    ax.expert_ffn_decode(pool, x, sel, w, y=y, workspace=ws)
    torch.cuda.synchronize()
    eager = y.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ax.expert_ffn_decode(pool, x, sel, w, y=y, workspace=ws, stream=s)
    torch.cuda.synchronize()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    assert ws.error_flags() == 0
