"""GPU parity of the reference's separable batch-pipeline steps, through the C-ABI, against the
pinned oracle (tests/test_oracle.py): affx_expert_gather_tokens and affx_expert_scatter_slots bit
for bit (index copies; per-token float sums in the same order), affx_expert_swiglu_quant with
the scales within 2 ulp and every E4M3 byte equal except where the device's expf moves a value
across a rounding boundary (a neighbouring code, at most 1 in 1000 bytes) -- shapes of a C4
prefill chunk's arenas (hidden 4096 / inter 2048, thousands of slots)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    from affinity_amd._lib import lib
    ax.init()
    return lib()


def _bf16(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_gather_tokens_bit_exact(lib, orc):
    rng = np.random.default_rng(21)
    dim, nb, nt = 4096, 96, 61
    src = rng.normal(0, 1, (dim, nb)).astype(np.float32)
    tok = rng.integers(0, nb, nt).astype(np.uint32)
    s, t = torch.from_numpy(src).cuda(), torch.from_numpy(tok).cuda()
    dst = torch.full((dim, nt), float("nan"), device="cuda")
    assert lib.affx_expert_gather_tokens(s.data_ptr(), dst.data_ptr(), t.data_ptr(), dim, nb, nt, None) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dst.cpu().numpy(), orc.gather_tokens(src, tok))


@pytest.mark.parametrize("nb_tok", [1, 7, 300])
def test_scatter_slots_bit_exact(lib, orc, nb_tok):
    rng = np.random.default_rng(22 + nb_tok)
    dim, nb_stride = 4096, nb_tok + 5
    counts = rng.integers(0, 7, nb_tok)
    counts[0] = max(counts[0], 1)
    if nb_tok > 2:
        counts[1] = 0                                     # a token without slots
    total = int(counts.sum())
    run = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    ordv = rng.permutation(total).astype(np.uint32)
    y = _bf16(rng.normal(0, 1, (dim, total)))
    block0 = rng.normal(0, 1, (dim, nb_stride)).astype(np.float32)
    want = orc.scatter_slots(y, block0.copy(), ordv, run, nb_tok)
    yd, od, rd = (torch.from_numpy(a).cuda() for a in (y.view(np.int16), ordv.view(np.int32), run.view(np.int32)))
    bd = torch.from_numpy(block0).cuda()
    assert lib.affx_expert_scatter_slots(yd.data_ptr(), bd.data_ptr(), od.data_ptr(), rd.data_ptr(), dim, nb_tok,
                                         nb_stride, total, None) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bd.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dim,total,weighted,limit", [(2048, 4000, True, 10.0), (4096, 70, False, 10.0),
                                                     (2048, 33, True, 0.0)])
def test_swiglu_quant_vs_oracle(lib, orc, dim, total, weighted, limit):
    rng = np.random.default_rng(23 + total)
    g = _bf16(rng.normal(0, 2.5, (dim, total)))
    u = _bf16(rng.normal(0, 2.5, (dim, total)))
    g[:128, 3] = 0                                         # an all-zero band of slot 3: scale 1
    u[:128, 3] = 0
    w = (0.05 + rng.random(total)).astype(np.float32) if weighted else None
    want_out, want_sc = orc.swiglu_quant(g, u, w, limit)
    gd, ud = (torch.from_numpy(a.view(np.int16)).cuda() for a in (g, u))
    wd = torch.from_numpy(w).cuda() if weighted else None
    out = torch.zeros((total, dim), dtype=torch.uint8, device="cuda")
    sc = torch.zeros((total, dim // 128), device="cuda")
    assert lib.affx_expert_swiglu_quant(gd.data_ptr(), ud.data_ptr(), wd.data_ptr() if weighted else None,
                                        out.data_ptr(), sc.data_ptr(), dim, total, limit, None) == 0
    torch.cuda.synchronize()
    got_out, got_sc = out.cpu().numpy(), sc.cpu().numpy()
    np.testing.assert_allclose(got_sc, want_sc, rtol=2.4e-7, atol=0)
    diff = got_out != want_out
    frac = diff.mean()
    # a differing byte is a neighbouring code of the same sign
    nb = np.abs(got_out[diff].astype(np.int32) - want_out[diff].astype(np.int32))
    print(f"swiglu_quant {dim}x{total}: {diff.sum()} of {diff.size} bytes differ ({frac:.2e})")
    assert frac <= 1e-3 and (nb <= 1).all()
    assert (got_out[3, :128] == 0).all() and got_sc[3, 0] == 1.0
