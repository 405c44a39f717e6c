"""GPU codebook producer parity: sample collection, the joint codebook fit, E4M3 projection,
packing and unpacking (src/quant/blockquant.cpp:252-492) against the reference's own fixtures
(small.npz, written by the compiled reference; c1_codebook.bin, the packed codebook of the config-1
recipe) and the oracle, bit for bit."""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
H, I = 4096, 2048


@pytest.fixture(scope="module")
def cbk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.codebook as cbk
    import affinity_amd.experts as ax
    ax.init()
    return cbk


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same(a, b, msg=""):
    """Bit for bit, except that any NaN matches any NaN (payloads are the platform's)."""
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    assert a.shape == b.shape, msg
    na, nb = np.isnan(a), np.isnan(b)
    np.testing.assert_array_equal(na, nb, err_msg=msg)
    np.testing.assert_array_equal(bits(a[~na]), bits(b[~nb]), err_msg=msg)


def gpu_fit(cbk, samples, iters=50, seed=1, flags=0):
    f = cbk.CodebookFit(samples.size)
    cb = f.fit(torch.from_numpy(np.ascontiguousarray(samples, np.float32)).cuda(), iters, seed, flags)
    return cb.cpu().numpy().reshape(-1), f.stats()


def test_collect_samples_matches_oracle(cbk, orc):
    rng = np.random.default_rng(3)
    for rows, cols, budget in ((64, 512, 4096), (100, 256, 1 << 22), (33, 200, 1000), (7, 64, 1), (128, 4096, 1 << 14)):
        w = (0.02 * rng.standard_normal((rows, cols))).astype(np.float32)
        w[1] = 0.0                       # a zero row
        w[2, 16:32] = 0.0                # a zero block
        w[4, :cols - cols % 16] = 0.0    # only the columns past the last block nonzero
        w[5, 3] = np.nan                 # NaN: ignored by the maxima, divided like any value
        got = cbk.collect_normalized_samples(torch.from_numpy(w).cuda(), budget).cpu().numpy()
        ref = orc.collect_samples(w, budget)
        same(got, ref, f"{rows}x{cols} budget {budget}")


def test_fit_matches_reference_fixture(cbk, small):
    s = small["fit_samples"]
    raw, (seq, passes) = gpu_fit(cbk, s, 50, 1)
    np.testing.assert_array_equal(bits(raw), bits(small["fit_cb_raw"]))
    proj = cbk.project_codebook_e4m3(torch.from_numpy(raw.copy()).cuda()).cpu().numpy()
    np.testing.assert_array_equal(bits(proj), bits(small["fit_cb_proj"]))
    assert passes > 0
    print(f"small fixture: {seq} sequential draws, {passes} Lloyd passes")


@pytest.mark.parametrize("n,iters,seed", [(16, 50, 1), (20, 5, 2), (64, 50, 3), (1000, 7, 4), (4101, 3, 5),
                                          (20000, 10, 9)])
def test_fit_matches_oracle(cbk, orc, n, iters, seed):
    # sizes below one block, below the 1024 entries (duplicate draws, an all-zero d2), ragged
    # tails (items outside a whole block), a single-block EM (an empty variant is reseeded)
    rng = np.random.default_rng(seed)
    s = np.clip(rng.standard_normal(n) * 0.4, -1, 1).astype(np.float32)
    raw, _ = gpu_fit(cbk, s, iters, seed)
    np.testing.assert_array_equal(bits(raw), bits(orc.fit_codebook(s, iters, seed)))


def test_fit_sequential_draws_give_the_same_codebook(cbk, small):
    s = small["fit_samples"][:24000]
    a, (seq_a, _) = gpu_fit(cbk, s, 8, 11)
    b, (seq_b, _) = gpu_fit(cbk, s, 8, 11, cbk.SEQUENTIAL_PICKS)
    assert seq_b == 1023
    np.testing.assert_array_equal(bits(a), bits(b))


def test_config1_codebook_on_gpu(cbk):
    """The config-1 recipe end to end on the GPU (weights from the GPU generator, 3 x 2^19 samples,
    fit_codebook(50, seed 1), projection, packing) reproduces the reference's packed codebook."""
    import affinity_amd.experts as ax
    mats = [ax.gen_normal(1000, I * H, 0.02).view(I, H), ax.gen_normal(1001, I * H, 0.02).view(I, H),
            ax.gen_normal(1002, H * I, 0.02).view(H, I)]
    s = torch.cat([cbk.collect_normalized_samples(m, 1 << 19) for m in mats])
    assert s.numel() == 3 * (1 << 19)
    f = cbk.CodebookFit(s.numel())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    cb = f.fit(s, 50, 1)
    e1.record()
    torch.cuda.synchronize()
    seq, passes = f.stats()
    print(f"config-1 fit: {e0.elapsed_time(e1):.1f} ms, {seq} sequential draws, {passes} Lloyd passes")
    packed = cbk.pack_codebook_e4m3_quads(cbk.project_codebook_e4m3(cb)).cpu().numpy().view(np.uint32)
    ref = np.fromfile(os.path.join(GOLDEN, "c1_codebook.bin"), dtype="<u4")
    np.testing.assert_array_equal(packed, ref)


def test_project_pack_unpack_match_oracle(cbk, orc, c1_codebook):
    rng = np.random.default_rng(1)
    cb = np.concatenate([rng.uniform(-2, 2, 6000), rng.standard_normal(1000) * 0.01,
                         [0.0, -0.0, 1.875, -1.875, 2.0, 100.0, -100.0, 1e-9, np.nan],
                         rng.uniform(-1, 1, 8192 - 7009)]).astype(np.float32)
    proj = cbk.project_codebook_e4m3(torch.from_numpy(cb.copy()).cuda()).cpu().numpy()
    same(proj, orc.project_codebook(cb))
    packed = cbk.pack_codebook_e4m3_quads(torch.from_numpy(cb).cuda()).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(packed, orc.pack_codebook(cb))
    un = cbk.unpack_codebook_e4m3_quads(torch.from_numpy(c1_codebook.view(np.int32)).cuda()).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(bits(un), bits(orc.unpack_codebook(c1_codebook)))


def test_producer_declines_and_limits(cbk):
    """The C-ABI's refusals and the collection's cap: weights are declined, a misaligned sample
    pointer and a short workspace are argument errors, and a collection into a buffer smaller
    than its count writes only `cap` floats while reporting the full count."""
    import ctypes as C
    from affinity_amd._lib import AFFX_DECLINED, AFFX_ERR_ARG, lib
    L = lib()
    s = torch.rand(4096, device="cuda")
    cb = torch.empty(8192, device="cuda")
    ws = torch.empty(int(L.affx_fit_codebook_workspace_size(4096)) + 256, dtype=torch.uint8, device="cuda")
    wsp = ws.data_ptr() + (-ws.data_ptr()) % 256
    n = int(L.affx_fit_codebook_workspace_size(4096))
    stream = torch.cuda.current_stream().cuda_stream
    assert L.affx_fit_codebook(s.data_ptr(), 4096, s.data_ptr(), 5, 1, 0, cb.data_ptr(), wsp, n, stream) == AFFX_DECLINED
    assert L.affx_fit_codebook(s.data_ptr() + 4, 4092, None, 5, 1, 0, cb.data_ptr(), wsp, n, stream) == AFFX_ERR_ARG
    assert L.affx_fit_codebook(s.data_ptr(), 4096, None, 5, 1, 0, cb.data_ptr(), wsp, n - 256, stream) == AFFX_ERR_ARG
    w = torch.randn(64, 256, device="cuda") * 0.02
    bound = int(L.affx_collect_samples_bound(64, 256, 1 << 20))
    assert bound == 64 * 256
    out = torch.full((bound,), -7.0, device="cuda")
    n_out = torch.zeros(1, dtype=torch.int64, device="cuda")
    cws = torch.empty(int(L.affx_collect_samples_workspace_size(64, 256, 1 << 20)), dtype=torch.uint8, device="cuda")
    cap = 1000   # not a multiple of 16: the block that would cross it is not written
    assert L.affx_collect_samples(w.data_ptr(), 64, 256, 1 << 20, out.data_ptr(), cap, n_out.data_ptr(),
                                  cws.data_ptr(), cws.numel(), stream) == 0
    full = cbk.collect_normalized_samples(w, 1 << 20)
    assert int(n_out.item()) == full.numel() == 64 * 256
    got = out.cpu().numpy()
    np.testing.assert_array_equal(bits(got[:992]), bits(full.cpu().numpy()[:992]))
    assert (got[992:] == -7.0).all()


def test_fit_at_quantizer_scale_matches_reference_fixture(cbk):
    """aff-quantize's scale (tools/aff_quantize.cpp:402-430 samples 24 matrices): 8 matrices of
    2^19 samples each, 4.2 M samples, fitted with fit_codebook(50, seed 1), against the raw
    codebook the compiled reference wrote for the same samples (tests/golden/fit_large.npz)."""
    import hashlib
    import affinity_amd.experts as ax
    f = np.load(os.path.join(GOLDEN, "fit_large.npz"))
    parts = []
    for i in range(8):
        rows, cols = (I, H) if i % 2 == 0 else (H, I)
        w = ax.gen_normal(3000 + i, rows * cols, 0.02).view(rows, cols)
        parts.append(cbk.collect_normalized_samples(w, 1 << 19))
        del w
    s = torch.cat(parts)
    assert s.numel() == int(f["n_samples"])
    assert hashlib.sha256(s.cpu().numpy().tobytes()).hexdigest() == str(f["samples_sha256"])
    fit = cbk.CodebookFit(s.numel())
    cb = fit.fit(s, 50, 1)
    seq, passes = fit.stats()
    print(f"quantizer-scale fit: {seq} sequential draws, {passes} Lloyd passes")
    np.testing.assert_array_equal(bits(cb.cpu().numpy().reshape(-1)), bits(f["cb_raw"]))
