"""GPU parity of the reference-shaped inner entry points (src/gpu/expert_kernel_hip.h):
affx_expert_ffn with expert_ffn_hip's arguments (a host array of per-matrix device pointers,
device route weights, caller scratch), against the layer-slab decode and the oracle."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import bf16_bits, planes, random_expert_container, rel_l2, slot_list

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


def _upload_matrix(lib, ex, lay, which, rows, cols, keep):
    """One matrix uploaded on its own, as aff-gpucheck does (tools/aff_gpucheck.cpp:54-74): its code
    and field planes permuted on the host by affx_matrix_to_device_layout, the row scales as they
    are, each in a buffer of its own."""
    from affinity_amd._lib import AffxMatrix
    c, f, r = planes(ex, lay, which)
    dc, df = np.zeros_like(c), np.zeros_like(f)
    assert lib().affx_matrix_to_device_layout(c.ctypes.data, f.ctypes.data, dc.ctypes.data, df.ctypes.data,
                                              rows, cols) == 0
    bufs = [torch.from_numpy(a.view(np.uint8).copy()).cuda() for a in (dc, df, r)]
    keep.extend(bufs)
    return AffxMatrix(bufs[0].data_ptr(), bufs[1].data_ptr(), bufs[2].data_ptr(), rows, cols)


# every n from one expert up (the reference's expert_ffn_hip takes any n >= 1 with its 2 * n *
# inter floats of scratch), at the benchmark shape and at inter 1024 (the smallest scratch)
@pytest.mark.parametrize("n,inter", [(1, 2048), (2, 2048), (5, 2048), (6, 2048), (16, 2048), (1, 1024), (3, 1024)])
def test_expert_ffn_pointer_table(ax, orc, c1_codebook, n, inter):
    from affinity_amd._lib import AffxDeviceExpert, lib, last_error
    hidden = 4096
    rng = np.random.default_rng(40 + n + inter)
    lay = ax.expert_layout(hidden, inter)
    ex = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n)])
    keep = []
    des = (AffxDeviceExpert * n)()
    for k in range(n):
        des[k].gate = _upload_matrix(lib, ex[k], lay, 0, inter, hidden, keep)
        des[k].up = _upload_matrix(lib, ex[k], lay, 1, inter, hidden, keep)
        des[k].down = _upload_matrix(lib, ex[k], lay, 2, hidden, inter, keep)
    cb = torch.from_numpy(c1_codebook.view(np.int32)).cuda()
    x = torch.from_numpy(rng.standard_normal(hidden).astype(np.float32)).cuda()
    w = torch.from_numpy((0.1 + 0.13 * np.arange(n)).astype(np.float32)).cuda()   # aff-gpucheck's weights
    y0 = torch.from_numpy(rng.standard_normal(hidden).astype(np.float32)).cuda()
    out = y0.clone()
    scratch = torch.empty(2 * n * inter, dtype=torch.float32, device="cuda")       # the reference's contract
    scratch.fill_(float("nan"))                                                     # no clearing needed
    assert lib().affx_expert_ffn(des, w.data_ptr(), n, cb.data_ptr(), x.data_ptr(), 10.0, scratch.data_ptr(),
                                 out.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0, last_error()
    torch.cuda.synchronize()
    # the layer-slab decode (staged launches) over the same experts in order: bit for bit
    pool = ax.ExpertPool.from_container(torch.from_numpy(ex.reshape(-1)).cuda(), c1_codebook, hidden, inter)
    sel = torch.arange(n, dtype=torch.int32, device="cuda").view(1, n)
    ys = ax.expert_ffn_decode(pool, x.view(1, hidden), sel, w.view(1, n), y=y0.clone().view(1, hidden),
                              accumulate=True, staged=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ys.view(hidden))
    ref = y0.cpu().numpy().copy()
    cbf = orc.unpack_codebook(c1_codebook)
    for k in range(n):
        orc.expert_ffn(np.ascontiguousarray(ex[k]), cbf, x.cpu().numpy(), float(w[k]), 10.0, ref, hidden, inter)
    err = rel_l2(out.cpu().numpy() - y0.cpu().numpy(), ref - y0.cpu().numpy())
    print(f"expert_ffn pointer table n={n}: rel_l2={err:.3e}")
    assert err <= TOL


def test_expert_ffn_declines_and_refuses_before_launching(ax, c1_codebook):
    """What the pointer-table form declines (more than 16 experts, hidden above 4096, no clamp
    limit) or refuses (a matrix of the wrong shape) is decided on the host: nothing is launched
    (the planes here are a small zero buffer that a launch would read past)."""
    from affinity_amd._lib import AffxDeviceExpert, AffxMatrix, lib, last_error
    hidden, inter = 4096, 2048
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    p = buf.data_ptr()
    e = AffxDeviceExpert()
    e.gate = AffxMatrix(p, p, p, inter, hidden)
    e.up = AffxMatrix(p, p, p, inter, hidden)
    e.down = AffxMatrix(p, p, p, hidden, inter)
    des17 = (AffxDeviceExpert * 17)(*([e] * 17))
    rc = lib().affx_expert_ffn(des17, p, 17, p, p, 10.0, p, p, None)
    assert rc == 1 and "at most" in last_error()
    wide = AffxDeviceExpert()
    wide.gate = AffxMatrix(p, p, p, inter, 2 * hidden)
    wide.up = AffxMatrix(p, p, p, inter, 2 * hidden)
    wide.down = AffxMatrix(p, p, p, 2 * hidden, inter)
    rc = lib().affx_expert_ffn((AffxDeviceExpert * 1)(wide), p, 1, p, p, 10.0, p, p, None)
    assert rc == 1 and "hidden" in last_error()
    rc = lib().affx_expert_ffn((AffxDeviceExpert * 1)(e), p, 1, p, p, 0.0, p, p, None)
    assert rc == 1 and "limit" in last_error()
    bad = AffxDeviceExpert()
    bad.gate, bad.up = e.gate, e.up
    bad.down = AffxMatrix(p, p, p, hidden, hidden)
    rc = lib().affx_expert_ffn((AffxDeviceExpert * 2)(e, bad), p, 2, p, p, 10.0, p, p, None)
    assert rc == -1 and "expected" in last_error()
    torch.cuda.synchronize()


def _grouped_slots(ax, pool, xb, lists, T, K):
    from affinity_amd._lib import lib, check
    start, tok, wt, ordv, run = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in lists)
    y = torch.zeros((T, pool.hidden), device="cuda")
    ws = ax.GroupedWorkspace(T, K, pool.n_experts, pool.hidden, pool.inter)
    L = pool.layer()
    check(lib().affx_expert_ffn_grouped_slots(C.byref(L), xb.data_ptr(), 0, T, start.data_ptr(), tok.data_ptr(),
                                              wt.data_ptr(), ordv.data_ptr(), run.data_ptr(), int(tok.numel()),
                                              y.data_ptr(), 0, ws.buf.data_ptr(), ws.bytes,
                                              torch.cuda.current_stream().cuda_stream), "grouped_slots")
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_grouped_slot_list(ax, orc, c1_codebook):
    """The slot-list prefill entry: on the list the routes entry builds itself it gives the same
    bits; on another valid list (each expert's slots in reverse token order, each token's slots
    reversed) it matches the oracle."""
    hidden, inter, n, T, K = 2048, 1024, 10, 300, 6
    rng = np.random.default_rng(91)
    lay = ax.expert_layout(hidden, inter)
    ex = np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n)])
    pool = ax.ExpertPool.from_container(torch.from_numpy(ex.reshape(-1)).cuda(), c1_codebook, hidden, inter)
    p = 1.0 / np.arange(1, n + 1) ** 1.1
    sel = np.stack([rng.choice(n, K, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    sel[4, 1] = 500   # padding
    w = rng.uniform(0.05, 1.0, (T, K)).astype(np.float32)
    x = bf16_bits(rng.standard_normal((T, hidden)).astype(np.float32))
    xb = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
    yr = ax.expert_ffn_grouped(pool, xb, torch.from_numpy(sel).cuda(), torch.from_numpy(w).cuda()).cpu().numpy()
    lists = slot_list(sel, w, n)
    ys = _grouped_slots(ax, pool, xb, lists, T, K)
    np.testing.assert_array_equal(ys.view(np.uint32), yr.view(np.uint32))
    start, tok, wt, ordv, run = lists
    remap = np.empty(tok.size, np.int64)
    for e in range(n):
        a, b = int(start[e]), int(start[e + 1])
        remap[a:b] = np.arange(b - 1, a - 1, -1)
    tok2, wt2 = np.empty_like(tok), np.empty_like(wt)
    tok2[remap], wt2[remap] = tok, wt
    ord2 = np.concatenate([remap[ordv[run[t]:run[t + 1]]][::-1] for t in range(T)]).astype(np.uint32)
    y2 = _grouped_slots(ax, pool, xb, (start, tok2, wt2, ord2, run), T, K)
    xr = (x.astype(np.uint32) << 16).view(np.float32)
    cbf = orc.unpack_codebook(c1_codebook)
    ref = np.zeros((T, hidden), np.float32)
    for t in range(T):
        for j in range(K):
            if sel[t, j] < n:
                orc.expert_ffn(np.ascontiguousarray(ex[sel[t, j]]), cbf, xr[t], float(w[t, j]), 10.0, ref[t], hidden, inter)
    err = rel_l2(y2, ref)
    print(f"slot list reordered rel_l2={err:.3e}")
    assert err <= TOL
