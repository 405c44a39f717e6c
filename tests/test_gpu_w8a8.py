"""GPU parity of the single-matrix W8A8 GEMM of the reference's batch pipeline
(affx_expert_gemm_w8a8 = expert_gemm_wmma_hip, src/gpu/expert_kernel_hip.h:217-228), through the
C-ABI, against the pinned oracle (tests/test_oracle.py): at the benchmark shapes (gate 2048 x 4096,
down 4096 x 2048), several tiles in one launch (64 listed tokens, one token, 37 tokens into a
strided arena whose other columns stay as they were, a pad), f32 and bf16 outputs. The block sums
are fp8 products summed by the MFMA, whose accumulation keeps about 2^-11.5 of a group's largest
product (pinned in tests/test_gpu_decode.py::test_mfma_fp8_accumulation_window); over random E4M3
bytes of the whole code range, as here, that measures about 5e-5 relative L2 against the oracle's
double sums. Held to 2e-4 (the expert-output bar is 1e-3); the bf16 outputs to one ulp of the value
plus that bound."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import planes, random_expert_container, rel_l2

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


@pytest.mark.parametrize("which,rows,cols,bf16", [(0, I, H, False), (2, H, I, False), (1, I, H, True)])
def test_expert_gemm_w8a8_matches_oracle(ax, orc, c1_codebook, which, rows, cols, bf16):
    from affinity_amd._lib import AffxExpertTile, AffxMatrix, last_error, lib
    rng = np.random.default_rng(500 + which + 10 * bf16)
    lay = ax.expert_layout(H, I)
    cbf = orc.unpack_codebook(c1_codebook)
    n_tok, ld2 = 150, 200
    x8 = rng.integers(0, 256, (n_tok, cols), dtype=np.uint8)
    x8[(x8 & 0x7F) == 0x7F] ^= 1                         # no NaN codes
    xs = rng.uniform(0.01, 2.0, (n_tok, cols // 128)).astype(np.float32)
    ydt = torch.int16 if bf16 else torch.float32
    # tiles: (expert, token ids or None, nt, output block, ld, column offset in it)
    tok0 = rng.choice(n_tok, 64, replace=False).astype(np.uint32)
    tok2 = rng.integers(0, n_tok, 37).astype(np.uint32)
    y0 = torch.zeros((rows, 64), dtype=ydt, device="cuda")
    y1 = torch.zeros((rows, 1), dtype=ydt, device="cuda")
    arena = torch.full((rows, ld2), 3, dtype=ydt, device="cuda")
    keep, exps = [], []
    tiles = (AffxExpertTile * 4)()
    spec = [(tok0, 64, y0, 0, 0), (None, 1, y1, 0, 0), (tok2, 37, arena, ld2, 100), (None, 0, None, 0, 0)]
    for e, (tok, nt, yb, ld, co) in enumerate(spec):
        ex = random_expert_container(rng, H, I, lay)
        exps.append(ex)
        c, f, r = planes(ex, lay, which)
        dc, df = np.zeros_like(c), np.zeros_like(f)
        assert lib().affx_matrix_to_device_layout(c.ctypes.data, f.ctypes.data, dc.ctypes.data, df.ctypes.data,
                                                  rows, cols) == 0
        bufs = [torch.from_numpy(a.view(np.uint8).copy()).cuda() for a in (dc, df, r)]
        td = torch.from_numpy(tok.view(np.int32)).cuda() if tok is not None else None
        keep.extend(bufs + ([td] if td is not None else []))
        esz = 2 if bf16 else 4
        tiles[e] = AffxExpertTile(bufs[0].data_ptr(), bufs[1].data_ptr(), bufs[2].data_ptr(),
                                  td.data_ptr() if td is not None else None,
                                  (yb.data_ptr() + co * esz) if yb is not None else None, nt, ld)
    tiles_d = torch.from_numpy(np.frombuffer(bytes(tiles), np.uint8).copy()).cuda()
    x8_d, xs_d = torch.from_numpy(x8).cuda(), torch.from_numpy(xs).cuda()
    cb = torch.from_numpy(c1_codebook.view(np.int32)).cuda()
    rc = lib().affx_expert_gemm_w8a8(tiles_d.data_ptr(), 4, 64, x8_d.data_ptr(), xs_d.data_ptr(), cb.data_ptr(),
                                     rows, cols, 0.5, int(bf16), None)
    assert rc == 0, last_error()
    torch.cuda.synchronize()

    def as_f32(t):
        a = t.cpu().numpy()
        return ((a.view(np.uint16).astype(np.uint32) << 16).view(np.float32) if bf16 else a)

    got_arena = as_f32(arena)
    for e, (tok, nt, yb, ld, co) in enumerate(spec[:3]):
        c, f, r = planes(exps[e], lay, which)
        ref = orc.expert_gemm_w8a8(c, f, r, tok, nt, x8, xs, cbf, rows, cols, 0.5, y_bf16=bf16)
        got = got_arena[:, co:co + nt] if ld else as_f32(yb)
        if bf16:
            # one bf16 ulp of the value, plus the f32 result's own error (near zero its sign may flip)
            rf = (ref.astype(np.uint32) << 16).view(np.float32)
            bound = np.abs(rf) * 2.0 ** -7 + 5e-4 * np.abs(rf).max()   # a bf16 ulp is 2^-8 to 2^-7 of the value
            over = (np.abs(got - rf) > bound).sum()
            print(f"w8a8 {rows}x{cols} tile {e} nt={nt}: bf16 outputs beyond one ulp + 5e-4 of the max: {over}")
            assert over == 0
        else:
            err = rel_l2(got, ref)
            worst = np.abs(got - ref).max() / np.abs(ref).max()
            print(f"w8a8 {rows}x{cols} tile {e} nt={nt}: rel_l2 {err:.3e}, worst/max {worst:.3e}")
            assert err <= 2e-4 and worst <= 5e-4
    # the arena's other columns are untouched
    untouched = np.concatenate([got_arena[:, :100], got_arena[:, 137:]], axis=1)
    three = ((np.full(1, 3, np.uint32) << 16).view(np.float32)[0]) if bf16 else 3.0
    assert (untouched == three).all()


def test_expert_gemm_w8a8_refusals(ax):
    """Shapes outside the layout and max_nt past the reference's 64 are declined, misaligned
    activations refused, before any launch; no tiles is a no-op."""
    from affinity_amd._lib import AFFX_DECLINED, lib
    x8 = torch.zeros((4, 1024), dtype=torch.uint8, device="cuda")
    xs = torch.ones((4, 8), device="cuda")
    cb = torch.zeros(2048, dtype=torch.int32, device="cuda")
    t = torch.zeros(64, dtype=torch.uint8, device="cuda")
    f = lib().affx_expert_gemm_w8a8
    assert f(t.data_ptr(), 0, 4, x8.data_ptr(), xs.data_ptr(), cb.data_ptr(), 16, 1024, 1.0, 0, None) == 0
    assert f(t.data_ptr(), 1, 65, x8.data_ptr(), xs.data_ptr(), cb.data_ptr(), 16, 1024, 1.0, 0, None) == AFFX_DECLINED
    assert f(t.data_ptr(), 1, 4, x8.data_ptr(), xs.data_ptr(), cb.data_ptr(), 24, 1024, 1.0, 0, None) == AFFX_DECLINED
    assert f(t.data_ptr(), 1, 4, x8.data_ptr(), xs.data_ptr(), cb.data_ptr(), 16, 1000, 1.0, 0, None) == AFFX_DECLINED
    assert f(t.data_ptr(), 1, 4, x8.data_ptr() + 4, xs.data_ptr(), cb.data_ptr(), 16, 1024, 1.0, 0, None) < 0
