"""The allocation-free decode entry (affx_expert_ffn_decode_noalloc) against the workspace entry
(affx_expert_ffn_decode), through the C-ABI: bit-identical outputs on calls in a row, each smaller
than the one before (the scratch array keeps the last call's contents); the call captured in a
HIP graph and replayed with new inputs, every replay bit-identical to the workspace decode and no
device memory taken; its status entry; and a clear refusal of a size beyond the array."""
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


def test_noalloc_decode_graph_replays_allocate_nothing(ax, c1_codebook):
    """The stated use: the call under graph capture. Static input buffers, three replays with new
    inputs copied in between (batch 1, the one-pass kernel, and M = 5), each replay equal bit for
    bit to the workspace decode of the same inputs; the device's free memory is the same before
    the first call and after the last replay (the entry allocates nothing); the status entry
    reports no give-up."""
    from affinity_amd._lib import last_error, lib
    hidden, inter, n, k = 4096, 2048, 256, 6
    pool = _pool(ax, c1_codebook, n, hidden, inter, seed=91)
    rng = np.random.default_rng(92)
    for M in (1, 5):
        x = torch.zeros((M, hidden), device="cuda")
        sel = torch.zeros((M, k), dtype=torch.int32, device="cuda")
        w = torch.zeros((M, k), device="cuda")
        y = torch.zeros((M, hidden), device="cuda")
        ws = ax.DecodeWorkspace(M, k, hidden, inter)
        want = torch.zeros((M, hidden), device="cuda")
        inputs = []
        for rep in range(4):
            inputs.append((torch.from_numpy((rng.standard_normal((M, hidden)) * 0.7).astype(np.float32)).cuda(),
                           torch.from_numpy(np.stack([rng.choice(n, k, replace=False) for _ in range(M)])
                                            .astype(np.int32)).cuda(),
                           torch.from_numpy(rng.uniform(0.05, 1.0, (M, k)).astype(np.float32)).cuda()))
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        # eager calls first (the entry's first call on a device may set up, outside capture)
        x.copy_(inputs[0][0]); sel.copy_(inputs[0][1]); w.copy_(inputs[0][2])
        for _ in range(3):
            assert _call_noalloc(pool, x, sel, w, y) == 0, last_error()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "an eager call of the allocation-free entry took device memory"
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            rc = _call_noalloc(pool, x, sel, w, y)
        assert rc == 0, last_error()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]   # (the instantiated graph's own memory excluded)
        for rep in range(1, 4):
            xi, si, wi = inputs[rep]
            x.copy_(xi); sel.copy_(si); w.copy_(wi)
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            ax.expert_ffn_decode(pool, xi, si, wi, y=want, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(y, want), (M, rep)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, "a replay took device memory"
        del g
        assert lib().affx_decode_noalloc_status(0, None) == 0, last_error()
        print(f"M={M}: three graph replays identical to the workspace decode, no device memory taken")
