"""GPU parity of the step after the routed experts: the FP8 shared expert (decode and batch forms)
against the oracle's restatement of the host composition (src/engine/model.cpp:1214-1222, its
matvec pinned to the reference's own matvec_dense in tests/test_oracle.py), and the
hyper-connection post bit for bit against the oracle's hc_expand (itself bit-identical to the
reference's, tests/test_oracle.py). Shapes are V4-Flash's: hidden 4096, inter 2048."""
import numpy as np
import pytest

from gpu_util import rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

H, I = 4096, 2048


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def fp8_matrix(rng, rows, cols):
    """E4M3 bytes over every non-NaN code, UE8M0 tile scales around 2^-7 (the reference decodes
    0x7F / 0xFF as NaN, which no trained weight holds)."""
    w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] ^= 1
    s = rng.integers(116, 124, ((rows + 127) // 128, (cols + 127) // 128), dtype=np.uint8)
    return w, s


@pytest.fixture(scope="module")
def shexp(ax):
    rng = np.random.default_rng(41)
    mats = [fp8_matrix(rng, I, H), fp8_matrix(rng, I, H), fp8_matrix(rng, H, I)]
    dev = [torch.from_numpy(a).cuda() for m in mats for a in m]
    return ax.SharedExpert(*dev), mats


def device_layout_np(w: np.ndarray) -> np.ndarray:
    """The dense FP8 device layout restated: 2 KiB per (16-row tile, 128-column step), [half][lane]
    [16 B], lane c + 16 kg holding row 16 tile + c, columns 128 step + 64 half + 16 kg .. + 15."""
    rows, cols = w.shape
    t = w.reshape(rows // 16, 16, cols // 128, 2, 4, 16)        # tile, c, step, half, kg, byte
    return np.ascontiguousarray(t.transpose(0, 2, 3, 4, 1, 5)).reshape(rows, cols)


def test_dense_device_layout(ax):
    """The GPU permutation equals the restatement byte for byte, and is a bijection (a matrix of
    distinct 32-bit indices comes back as a permutation of itself)."""
    rng = np.random.default_rng(2)
    for rows, cols in ((16, 128), (2048, 4096), (4096, 2048), (48, 384)):
        w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        got = ax.dense_fp8_to_device_layout(torch.from_numpy(w).cuda()).cpu().numpy()
        np.testing.assert_array_equal(got, device_layout_np(w))
    idx = np.arange(64 * 512, dtype=np.uint32).view(np.uint8).reshape(64, 2048)
    got = ax.dense_fp8_to_device_layout(torch.from_numpy(idx).cuda()).cpu().numpy()
    # (the layout moves 16-byte chunks, so 4-byte indices stay whole: every index appears once)
    assert np.array_equal(np.sort(np.ascontiguousarray(got).view(np.uint32).reshape(-1)),
                          np.arange(64 * 512, dtype=np.uint32))


def oracle_rows(orc, mats, x):
    (wg, sg), (wu, su), (wd, sd) = mats
    return np.stack([orc.shared_expert(wg, sg, wu, su, wd, sd, np.ascontiguousarray(x[t]), 10.0)
                     for t in range(x.shape[0])])


@pytest.mark.parametrize("M", [1, 3, 5, 6, 8])
def test_shared_decode_matches_oracle(ax, orc, shexp, M):
    """M tokens, added into a block that already holds the routed sum: the addition is exact
    f32 (the block afterwards minus before is the shared expert's output)."""
    S, mats = shexp
    rng = np.random.default_rng(100 + M)
    x = rng.standard_normal((M, H)).astype(np.float32)
    y0 = (rng.standard_normal((M, H)) * 0.01).astype(np.float32)
    gx, gy = torch.from_numpy(x).cuda(), torch.from_numpy(y0).cuda()
    S.decode(gx, gy, accumulate=True)
    got = gy.cpu().numpy()
    ref = oracle_rows(orc, mats, x)
    err = rel_l2(got - y0, ref)
    print(f"shared decode M={M}: rel_l2={err:.3e}")
    assert err <= 1e-3
    # stored form equals the accumulated contribution's recomputation
    gy2 = torch.full((M, H), 7.0, device="cuda")
    S.decode(gx, gy2, accumulate=False)
    assert rel_l2(gy2.cpu().numpy(), ref) <= 1e-3


def test_shared_decode_dim_major_arena(ax, orc, shexp):
    """The engine's dim-major arenas: x and the block [hidden][nb] with nb = 8 slots, 6 live."""
    S, mats = shexp
    rng = np.random.default_rng(7)
    nb, M = 8, 6
    x = rng.standard_normal((H, nb)).astype(np.float32)
    gx = torch.from_numpy(x).cuda()
    gy = torch.zeros((H, nb), device="cuda")
    S.decode(gx.t()[:M], gy.t()[:M], accumulate=True)   # (token stride 1, dim stride nb)
    got = gy.cpu().numpy().T[:M]
    ref = oracle_rows(orc, mats, np.ascontiguousarray(x.T[:M]))
    assert rel_l2(got, ref) <= 1e-3
    assert not gy.cpu().numpy()[:, M:].any()    # slots past M untouched


# The batch's two forms: "lib", the default (weights widened to bf16, hipBLASLt GEMMs in f32, the
# SwiGLU output as two bf16 terms: about 16 significant bits everywhere), and "mfma", the fp8 MFMA
# kernels (activations as E4M3 terms) that run where the library declines a shape.
BATCH_TOL = {"lib": 2e-5, "mfma": 1e-3}


@pytest.fixture(params=["lib", "mfma"])
def form(request, monkeypatch):
    if request.param == "mfma":
        monkeypatch.setenv("AFFX_SHARED_BATCH", "mfma")
    else:
        monkeypatch.delenv("AFFX_SHARED_BATCH", raising=False)
    return request.param


@pytest.mark.parametrize("T,lo", [(200, False), (200, True), (61, True), (1, False)])
def test_shared_batch_matches_oracle(ax, orc, shexp, T, lo, form):
    S, mats = shexp
    rng = np.random.default_rng(300 + T + lo)
    xf = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).cuda()
    xh = xf.to(torch.bfloat16)
    xl = (xf - xh.float()).to(torch.bfloat16) if lo else None
    xr = (xh.float() + (xl.float() if lo else 0)).cpu().numpy()
    y0 = torch.from_numpy((rng.standard_normal((T, H)) * 0.01).astype(np.float32)).cuda()
    y = y0.clone()
    S.batch(xh, y, x_lo=xl, accumulate=True)
    ref = oracle_rows(orc, mats, xr)
    err = rel_l2((y - y0).cpu().numpy(), ref)
    print(f"shared batch T={T} lo={lo} {form}: rel_l2={err:.3e}")
    assert err <= BATCH_TOL[form]


def test_shared_batch_prefill_shape_sampled(ax, orc, shexp, form):
    """The C4 prefill chunk (4096 tokens): 24 sampled tokens against the oracle, including the
    first and last token tiles of the MFMA form's GEMMs (96 and 60 tokens a tile). y starts as NaN:
    a stored (not accumulated) result must not read it."""
    S, mats = shexp
    T = 4096
    g = torch.Generator(device="cuda").manual_seed(9)
    xh = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.full((T, H), float("nan"), device="cuda")
    S.batch(xh, y, accumulate=False)
    assert not torch.isnan(y).any()
    pick = np.array([0, 1, 95, 96, 97, 1000, 2047, 2048, 3000, 4000, 4031, 4032, 4033, 4090, 4094, 4095,
                     17, 333, 777, 1234, 2500, 3333, 3700, 3999])
    ref = oracle_rows(orc, mats, xh.float().cpu().numpy()[pick])
    err = rel_l2(y.cpu().numpy()[pick], ref)
    print(f"shared batch T=4096 (24 sampled) {form}: rel_l2={err:.3e}")
    assert err <= BATCH_TOL[form]


def test_shared_batch_graph_replay(ax, shexp, form):
    """The batch captured in a HIP graph (after an eager call of the same token count, which
    resolves the library GEMM's plan outside the capture) and replayed three times on new inputs,
    with eager work between the replays: every replay equals the eager call on the same inputs
    bit for bit (the library GEMM records one kernel launch per GEMM and no memset)."""
    S, _ = shexp
    T = 300
    g = torch.Generator(device="cuda").manual_seed(23)
    xs = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ys = torch.zeros((T, H), device="cuda")
    xs.copy_(torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16))
    S.batch(xs, ys, accumulate=False)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        S.batch(xs, ys, accumulate=False)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        S.batch(xs, ys, accumulate=False)
    for rep in range(3):
        xn = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
        want = S.batch(xn, torch.zeros((T, H), device="cuda"), accumulate=False)
        xs.copy_(xn)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, want), f"replay {rep} differs from the eager call"


def test_shared_declines(ax, shexp):
    from affinity_amd._lib import AffxDeclined, AffxError
    S, _ = shexp
    x = torch.zeros((9, H), device="cuda")
    with pytest.raises(AffxDeclined):
        S.decode(x, torch.zeros_like(x))             # 9 tokens: the batch form's job
    import ctypes
    from affinity_amd._lib import AFFX_DECLINED, check, lib
    y = torch.zeros((1, H), device="cuda")
    ws = torch.empty(lib().affx_shared_decode_workspace_size(1, H, I), dtype=torch.uint8, device="cuda")
    bad = type(S.abi).from_buffer_copy(S.abi)
    bad.swiglu_limit = 0.0                           # the reference's "no clamp"
    rc = lib().affx_shared_expert_decode(ctypes.byref(bad), x.data_ptr(), H, 1, 1, y.data_ptr(), H, 1, 0,
                                         ws.data_ptr(), ws.numel(), 0)
    assert rc == AFFX_DECLINED
    bad = type(S.abi).from_buffer_copy(S.abi)
    bad.down.rows = H - 1                            # shapes that do not chain
    with pytest.raises(AffxError):
        check(lib().affx_shared_expert_decode(ctypes.byref(bad), x.data_ptr(), H, 1, 1, y.data_ptr(), H, 1, 0,
                                              ws.data_ptr(), ws.numel(), 0), "decode")
    with pytest.raises(AffxError):                   # workspace too small
        check(lib().affx_shared_expert_decode(ctypes.byref(S.abi), x.data_ptr(), H, 1, 1, y.data_ptr(), H, 1, 0,
                                              ws.data_ptr(), 16, 0), "decode")
    # the batch: a workspace off 16-byte alignment, and one too small, are refused before any launch
    xb = torch.zeros((4, H), dtype=torch.bfloat16, device="cuda")
    yb = torch.zeros((4, H), device="cuda")
    wsb = torch.empty(lib().affx_shared_batch_workspace_size(4, H, I) + 256, dtype=torch.uint8, device="cuda")
    for ptr, n in ((wsb.data_ptr() + 8, wsb.numel() - 8), (wsb.data_ptr(), 1024)):
        with pytest.raises(AffxError):
            check(lib().affx_shared_expert_batch(ctypes.byref(S.abi), xb.data_ptr(), 0, 4, yb.data_ptr(), 0, ptr, n,
                                                 0), "batch")


@pytest.mark.parametrize("n_hc", [1, 2, 4, 8])
def test_hc_post_bit_exact(ax, orc, n_hc):
    rng = np.random.default_rng(n_hc)
    hc = rng.standard_normal((n_hc, H)).astype(np.float32)
    blk = rng.standard_normal(H).astype(np.float32)
    post = rng.standard_normal(n_hc).astype(np.float32)
    comb = rng.standard_normal(n_hc * n_hc).astype(np.float32)
    gb = torch.from_numpy(blk).cuda()
    out = ax.hc_post(gb, torch.from_numpy(hc).cuda(), torch.from_numpy(post).cuda(), torch.from_numpy(comb).cuda())
    ref = orc.hc_expand(blk, hc, post, comb)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert not gb.cpu().numpy().any()          # the block is left zero


def test_hc_add_and_declines(ax, orc):
    from affinity_amd._lib import AffxDeclined
    rng = np.random.default_rng(5)
    hc = rng.standard_normal((1, H)).astype(np.float32)
    blk = rng.standard_normal(H).astype(np.float32)
    ghc, gb = torch.from_numpy(hc).cuda(), torch.from_numpy(blk).cuda()
    ax.hc_post(gb, ghc, None, None, zero_block=False)
    assert np.array_equal(ghc.cpu().numpy()[0], orc.hc_add(hc[0], blk))
    assert np.array_equal(gb.cpu().numpy(), blk)   # zero_block = 0 keeps it
    with pytest.raises(AffxDeclined):
        z = torch.zeros((3, H), device="cuda")
        ax.hc_post(gb, z, torch.zeros(3, device="cuda"), torch.zeros(9, device="cuda"))


@pytest.mark.parametrize("n_hc", [1, 4, 8])
def test_hc_post_batch_bit_exact(ax, orc, n_hc):
    """Dim-major bf16 arenas of nb = 37 tokens: every token against the oracle's hc_expand on the
    same bf16 inputs, rounded to bf16 once."""
    rng = np.random.default_rng(20 + n_hc)
    nb = 37
    hcf = torch.from_numpy(rng.standard_normal((n_hc, H, nb)).astype(np.float32))
    hcb = hcf.to(torch.bfloat16)
    blk = rng.standard_normal((H, nb)).astype(np.float32)
    post = rng.standard_normal((n_hc, nb)).astype(np.float32)
    comb = rng.standard_normal((n_hc * n_hc, nb)).astype(np.float32)
    gb = torch.from_numpy(blk).cuda()
    out = ax.hc_post_batch(gb, hcb.cuda(), torch.from_numpy(post).cuda(), torch.from_numpy(comb).cuda())
    got = out.cpu().view(torch.int16).numpy().astype(np.uint16)
    hin = hcb.float().numpy()
    for b in range(nb):
        ref = orc.hc_expand(blk[:, b].copy(), np.ascontiguousarray(hin[:, :, b]), post[:, b].copy(),
                            comb[:, b].copy())
        rb = np.array([orc.f32_to_bf16(float(v)) for v in ref.reshape(-1)], np.uint16).reshape(n_hc, H)
        assert np.array_equal(got[:, :, b], rb), f"token {b}"
    assert not gb.cpu().numpy().any()
    # no control: lane 0 += block, rounded to bf16
    hc0 = hcb[0].cuda().contiguous()
    gb = torch.from_numpy(blk).cuda()
    ax.hc_post_batch(gb, hc0.view(1, H, nb), None, None)
    want = (hcb[0].float() + torch.from_numpy(blk)).to(torch.bfloat16)
    assert torch.equal(hc0.cpu(), want)
    assert not gb.cpu().numpy().any()
