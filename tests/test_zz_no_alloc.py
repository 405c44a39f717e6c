"""The allocation-free decode entry (affx_expert_ffn_decode_noalloc) against the workspace entry
(affx_expert_ffn_decode), through the C-ABI: bit-identical outputs on two calls in a row, the
second smaller than the first (the scratch array keeps the last call's contents), and a clear
refusal of a size beyond the array."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def _pool(ax, c1_codebook, n, hidden, inter, seed):
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


def _call_noalloc(pool, x, sel, w, y, accumulate=False):
    from affinity_amd._lib import lib
    L = pool.layer()
    M, hidden = x.shape
    return lib().affx_expert_ffn_decode_noalloc(C.byref(L), x.data_ptr(), x.stride(0), 1, M, sel.data_ptr(),
                                                w.data_ptr(), sel.shape[1], y.data_ptr(), y.stride(0), 1,
                                                int(accumulate), torch.cuda.current_stream().cuda_stream)


def test_noalloc_decode_equals_workspace_decode(ax, c1_codebook):
    from affinity_amd._lib import last_error
    hidden, inter, n, k = 4096, 2048, 256, 6
    pool = _pool(ax, c1_codebook, n, hidden, inter, seed=77)
    rng = np.random.default_rng(78)
    for call, M in enumerate((8, 2, 1)):   # each call smaller than the one before
        x = torch.from_numpy((rng.standard_normal((M, hidden)) * 0.7).astype(np.float32)).cuda()
        sel = torch.from_numpy(np.stack([rng.choice(n, k, replace=False) for _ in range(M)]).astype(np.int32)).cuda()
        w = torch.from_numpy(rng.uniform(0.05, 1.0, (M, k)).astype(np.float32)).cuda()
        y0 = torch.from_numpy(rng.standard_normal((M, hidden)).astype(np.float32)).cuda()
        want = ax.expert_ffn_decode(pool, x, sel, w, y=y0.clone(), accumulate=True,
                                    workspace=ax.DecodeWorkspace(M, k, hidden, inter))
        got = y0.clone()
        assert _call_noalloc(pool, x, sel, w, got, accumulate=True) == 0, last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (call, M)
        print(f"call {call}: M={M} identical")


def test_noalloc_decode_refuses_oversize(ax, c1_codebook):
    from affinity_amd._lib import AFFX_ERR_ARG, last_error
    hidden, inter, n = 1024, 1024, 16
    pool = _pool(ax, c1_codebook, n, hidden, inter, seed=3)
    x = torch.zeros((8, hidden), device="cuda")
    sel = torch.zeros((8, 9), dtype=torch.int32, device="cuda")   # 72 routes > 64
    w = torch.zeros((8, 9), device="cuda")
    y = torch.zeros((8, hidden), device="cuda")
    assert _call_noalloc(pool, x, sel, w, y) == AFFX_ERR_ARG
    assert "exceed the scratch array" in last_error()
