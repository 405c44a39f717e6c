"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked against at least one of:
  * golden vectors the compiled reference wrote (tests/golden/*, make_golden.py);
  * the reference library itself (oracle/_ref/libaffref.so) on fresh inputs, where it was built;
  * closed forms and invariants fixed by the mathematics or the format.
"""
import hashlib
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
H, I = 4096, 2048


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def ref():
    from oracle import load_ref, ref_available
    if not ref_available():
        pytest.skip("reference library not built here (needs the reference tree)")
    return load_ref()


@pytest.fixture(scope="module")
def manifest():
    return json.load(open(os.path.join(GOLDEN, "c1_manifest.json")))


# ---------------------------------------------------------------------------------------------
# element codecs
# ---------------------------------------------------------------------------------------------

def test_e4m3_closed_form_and_reference(orc, scalars):
    got = np.array([orc.e4m3_to_float(b) for b in range(256)], np.float32)
    b = np.arange(256)
    e, m, s = (b >> 3) & 15, b & 7, np.where(b & 0x80, -1.0, 1.0)
    closed = s * np.where(e == 0, m * 2.0 ** -9, (8 + m) * 2.0 ** (e - 10.0))
    nan = (b & 0x7F) == 0x7F
    np.testing.assert_array_equal(got[~nan], closed[~nan].astype(np.float32))
    assert np.isnan(got[nan]).all() and nan.sum() == 2
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], scalars["e4m3"].view(np.uint32)[~nan])
    assert got[0x7E] == 448.0 and got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9


def test_bf16_rne_reference_and_nearest_even(orc, scalars):
    f = scalars["bf_in"]
    got = np.array([orc.f32_to_bf16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, scalars["bf_out"])
    # nearest with ties to even, for finite values whose result stays finite
    for v, h in zip(f[:2000], got[:2000]):
        u = np.float32(v).view(np.uint32)
        lo = np.uint32(u & 0xFFFF0000)
        hi = np.uint32(lo + 0x10000)
        dlo = abs(float(np.float32(v)) - float(lo.view(np.float32)))
        dhi = abs(float(hi.view(np.float32)) - float(np.float32(v)))
        r = int(h) << 16
        if not np.isfinite(hi.view(np.float32)):
            continue
        if dlo < dhi:
            assert r == lo
        elif dhi < dlo:
            assert r == hi
        else:
            assert (r >> 16) % 2 == 0


def test_bit_streams_lsb_first(orc):
    buf = np.zeros(8, np.uint8)
    orc.lib.orc_pack_bits(buf.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_uint8)), 0, 10, 0x3A5)
    assert buf[0] == 0xA5 and buf[1] == 0x03
    rng = np.random.default_rng(0)
    vals = rng.integers(0, 1 << 10, 200)
    s = np.zeros(250, np.uint8)
    import ctypes as C
    p = s.ctypes.data_as(C.POINTER(C.c_uint8))
    for i, v in enumerate(vals):
        orc.lib.orc_pack_bits(p, i, 10, int(v))
    # closed form: value i occupies stream bits 10i..10i+9, LSB first
    bits = np.unpackbits(s, bitorder="little")
    for i, v in enumerate(vals):
        assert int(sum(int(bits[10 * i + j]) << j for j in range(10))) == v
        assert orc.lib.orc_unpack_bits(p, i, 10) == v


# ---------------------------------------------------------------------------------------------
# synthetic generator
# ---------------------------------------------------------------------------------------------

def _splitmix_np(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        k = np.arange(1, n + 1, dtype=np.uint64)
        x = np.uint64(seed) + k * np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def test_splitmix64_known_answers(orc):
    # published first outputs of splitmix64 from seed 0 (Vigna's reference implementation)
    assert [orc.splitmix_at(0, k) for k in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                                        0x06C45D188009454F]
    np.testing.assert_array_equal(_splitmix_np(12345, 1000),
                                  np.array([orc.splitmix_at(12345, k) for k in range(1000)], np.uint64))


def test_generator_is_box_muller_bf16(orc, manifest):
    n = 200_000
    d = _splitmix_np(1000, 2 * n)
    u1 = ((d[0::2] >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = ((d[1::2] >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
    np.testing.assert_allclose(orc.normal_f64(1000, n), z, rtol=1e-14, atol=1e-14)
    f = (0.02 * z).astype(np.float32).view(np.uint32).astype(np.uint64)
    bf = (((f + 0x7FFF + ((f >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(orc.normal_bf16(1000, n, 0.02), bf)
    # and the config-1 inputs the reference was run on
    assert sha(orc.normal_bf16(7, H, 1.0)) == manifest["inputs"]["x"]


# ---------------------------------------------------------------------------------------------
# geometry
# ---------------------------------------------------------------------------------------------

def test_expert_layout_closed_form(orc):
    stride, off, size = orc.expert_layout(H, I)
    assert stride == 9_060_352
    assert list(off) == [0, 7_864_320, 9_043_968, 2_621_440, 8_257_536, 9_048_064, 5_242_880,
                         8_650_752, 9_052_160]
    assert list(size[:3]) == [I * H * 10 // 32, I * H * 6 // 128, I * 2]


def test_expert_layout_matches_reference(orc, ref):
    for h, i in ((4096, 2048), (1024, 1024), (7168, 2048), (4096, 1536)):
        s, o, z = orc.expert_layout(h, i)
        rs, ro, rz = ref.expert_layout(h, i)
        assert s == rs and list(o) == list(ro) and list(z) == list(rz)


# ---------------------------------------------------------------------------------------------
# codebook fit
# ---------------------------------------------------------------------------------------------

def test_collect_samples_closed_form(orc):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((64, 128)).astype(np.float32)
    w[16] = 0.0
    w[32, :16] = 0.0
    s = orc.collect_samples(w, 64 * 128 // 16)   # stride 16: rows 0, 16, 32, 48
    exp = []
    for r in (0, 32, 48):                        # row 16 is all zero
        for b in range(8):
            blk = w[r, 16 * b:16 * b + 16]
            m = np.abs(blk).max()
            if m > 0:
                exp.append(blk / m)
    np.testing.assert_array_equal(s, np.concatenate(exp).astype(np.float32))


def test_collect_samples_matches_reference(orc, ref):
    rng = np.random.default_rng(2)
    for rows, cols, budget in ((100, 64, 1000), (256, 512, 1 << 12), (33, 4096, 1 << 20)):
        w = rng.standard_normal((rows, cols)).astype(np.float32)
        np.testing.assert_array_equal(orc.collect_samples(w, budget), ref.collect_samples(w, budget))


def test_fit_small_matches_reference_fixture(orc, small):
    s = small["fit_samples"]
    raw = orc.fit_codebook(s, 50, 1)
    np.testing.assert_array_equal(raw.view(np.uint32), small["fit_cb_raw"].view(np.uint32))
    np.testing.assert_array_equal(orc.project_codebook(raw).view(np.uint32),
                                  small["fit_cb_proj"].view(np.uint32))


def test_fit_matches_reference_other_seeds(orc, ref):
    rng = np.random.default_rng(3)
    s = (rng.standard_normal(4 * 4 * 3000) * 0.3).astype(np.float32)
    for seed, iters in ((1, 50), (9, 7)):
        a = orc.fit_codebook(s, iters, seed)
        b = ref.fit_codebook(s, iters, seed, project=False)
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_projection_is_nearest_restricted_e4m3(orc):
    tbl = np.array([orc.e4m3_to_float(b) for b in range(256)], np.float32)
    allowed = np.array([((b >> 3) & 15) in range(1, 8) and (b & 0x7F) != 0x7F for b in range(256)])
    rng = np.random.default_rng(4)
    xs = np.concatenate([rng.uniform(-2.5, 2.5, 3000), [0.0, -0.0, 1e-9, 2.0, -1.875, 1.9375]]).astype(np.float32)
    for x in xs:
        b = orc.e4m3_nearest(float(x))
        assert allowed[b]
        d = np.abs(tbl[allowed] - x)
        assert abs(tbl[b] - x) == d.min()
        # ties resolve to the lowest byte
        assert b == np.flatnonzero(allowed)[np.argmin(d)]


def test_config1_codebook_matches_reference(orc):
    """The full config-1 recipe (3 x 2^19 samples, fit_codebook(50, seed 1), projection, pack)
    reproduces the reference's packed codebook bit for bit."""
    wg = orc.normal_bf16(1000, I * H, 0.02).reshape(I, H)
    wu = orc.normal_bf16(1001, I * H, 0.02).reshape(I, H)
    wd = orc.normal_bf16(1002, H * I, 0.02).reshape(H, I)
    s = np.concatenate([orc.collect_samples(w, 1 << 19) for w in (wg, wu, wd)])
    assert s.size == 3 * (1 << 19)
    cb = orc.project_codebook(orc.fit_codebook(s, 50, 1))
    packed = np.fromfile(os.path.join(GOLDEN, "c1_codebook.bin"), dtype="<u4")
    np.testing.assert_array_equal(orc.pack_codebook(cb), packed)
    assert orc.codebook_exponents_ok(packed)
    np.testing.assert_array_equal(orc.unpack_codebook(packed).view(np.uint32), cb.view(np.uint32))


# ---------------------------------------------------------------------------------------------
# quantise / dequantise
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["a", "b", "c", "d"])
def test_quantize_matches_reference_fixture(orc, small, c1_codebook, case):
    cb = orc.unpack_codebook(c1_codebook)
    w = small[f"{case}_w"]
    c, f, r = orc.quantize(w, cb)
    np.testing.assert_array_equal(c, small[f"{case}_codes"])
    np.testing.assert_array_equal(f, small[f"{case}_fields"])
    np.testing.assert_array_equal(r, small[f"{case}_rs"])
    # the reference's acceleration grid is exact: same bytes as its plain scan
    np.testing.assert_array_equal(small[f"{case}_codes"], small[f"{case}_codes_nosearch"])
    np.testing.assert_array_equal(small[f"{case}_fields"], small[f"{case}_fields_nosearch"])
    ci, fi, _ = orc.quantize(w, cb, small[f"{case}_imp"])
    np.testing.assert_array_equal(ci, small[f"{case}_codes_imp"])
    np.testing.assert_array_equal(fi, small[f"{case}_fields_imp"])
    # uniform importance gives the bytes of no importance
    c1, f1, _ = orc.quantize(w, cb, np.ones(w.shape[1], np.float32))
    np.testing.assert_array_equal(c1, c)
    np.testing.assert_array_equal(f1, f)


def test_quantize_matches_reference_random(orc, ref, c1_codebook):
    cb = orc.unpack_codebook(c1_codebook)
    rng = np.random.default_rng(5)
    for rows, cols in ((7, 128), (16, 1024)):
        w = (rng.standard_normal((rows, cols)) * rng.uniform(0.001, 0.1, (rows, 1))).astype(np.float32)
        w[0, :16] = 0
        a = orc.quantize(w, cb)
        b = ref.quantize(w, cb, None, search=True)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


@pytest.fixture(scope="module")
def c1_planes(orc, c1_codebook):
    cb = orc.unpack_codebook(c1_codebook)
    mats = {"gate": orc.normal_bf16(1000, I * H, 0.02).reshape(I, H),
            "up": orc.normal_bf16(1001, I * H, 0.02).reshape(I, H),
            "down": orc.normal_bf16(1002, H * I, 0.02).reshape(H, I)}
    return cb, {k: orc.quantize(w, cb) for k, w in mats.items()}


def test_config1_planes_match_reference(c1_planes, manifest):
    _, q = c1_planes
    for name in ("gate", "up", "down"):
        for i, k in enumerate(("codes", "fields", "rscales")):
            assert sha(q[name][i]) == manifest["planes"][name][k], (name, k)
        rows = manifest["rows"][name]
        for r, want in rows.items():
            r = int(r)
            cols = H if name != "down" else I
            cb_row, f_row = cols * 10 // 32, cols * 6 // 128
            assert q[name][0][r * cb_row:(r + 1) * cb_row].tobytes().hex() == want["codes"]
            assert q[name][1][r * f_row:(r + 1) * f_row].tobytes().hex() == want["fields"]
            assert int(q[name][2][r]) == want["rscale"]


def test_config1_dequant_and_ffn_match_reference(orc, c1_planes, manifest):
    cb, q = c1_planes
    dims = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    for name in ("gate", "up", "down"):
        assert sha(orc.dequantize(*q[name], *dims[name], cb)) == manifest["dequant"][name]
    x = orc.normal_bf16(7, H, 1.0)
    g = orc.gemv(*q["gate"], I, H, cb, x)
    u = orc.gemv(*q["up"], I, H, cb, x)
    a = orc.swiglu(g, u, 10.0)
    y = orc.gemv(*q["down"], H, I, cb, a, 1.0)
    assert sha(g) == manifest["ffn"]["g"] and sha(u) == manifest["ffn"]["u"]
    assert sha(a) == manifest["ffn"]["a"] and sha(y) == manifest["ffn"]["y"]
    np.testing.assert_array_equal(y, np.fromfile(os.path.join(GOLDEN, "c1_ffn_y.bin"), dtype="<f4"))


def _c1_container(orc, q):
    """The config-1 expert in container layout: the nine planes at orc_expert_layout's offsets."""
    stride, off, size = orc.expert_layout(H, I)
    ex = np.zeros(stride, np.uint8)
    for m, name in enumerate(("gate", "up", "down")):
        for p in range(3):
            b = np.ascontiguousarray(q[name][p]).view(np.uint8).reshape(-1)
            assert b.size == size[3 * m + p]
            ex[off[3 * m + p]:off[3 * m + p] + b.size] = b
    return ex


def test_config1_expert_ffn_matches_reference(orc, c1_planes):
    """orc_expert_ffn, the checker of every GPU FFN test, reproduces the reference-written config-1
    output bit for bit from the container expert (plane order, where the route weight is applied,
    the clamp: src/engine/model.cpp:1187-1198 over expert_gemv_scaled_mt and swiglu). With a
    route weight w and a nonzero y it adds w * tmp per element, as expert_gemv_scaled does
    (src/engine/expert_kernel.cpp:126-139)."""
    cb, q = c1_planes
    ex = _c1_container(orc, q)
    x = orc.normal_bf16(7, H, 1.0)
    fixture = np.fromfile(os.path.join(GOLDEN, "c1_ffn_y.bin"), dtype="<f4")
    y = orc.expert_ffn(ex, cb, x, 1.0, 10.0)
    np.testing.assert_array_equal(y.view(np.uint32), fixture.view(np.uint32))
    y0 = np.linspace(-3, 3, H).astype(np.float32)
    y2 = orc.expert_ffn(ex, cb, x, 0.375, 10.0, y0.copy())
    np.testing.assert_array_equal(y2.view(np.uint32), (y0 + np.float32(0.375) * fixture).view(np.uint32))


def _numpy_dequant(codes, fields, rs, rows, cols, cb):
    """Independent statement of the format: 10-bit codes and 6-bit fields LSB-first; field bits
    [0..2] s, [3] sign, [4] rotate, [5] variant; w = rs * 2^s * (+-1) * e[v][code][(p+rh)%4]."""
    cbits = np.unpackbits(codes, bitorder="little").reshape(-1, 10)
    fbits = np.unpackbits(fields, bitorder="little").reshape(-1, 6)
    code = (cbits * (1 << np.arange(10))).sum(1).reshape(rows, cols // 16, 4)
    f = (fbits * (1 << np.arange(6))).sum(1).reshape(rows, cols // 16)
    s, sign, rot, var = f & 7, (f >> 3) & 1, (f >> 4) & 1, f >> 5
    e = cb.reshape(2, 1024, 4)[var[:, :, None], code]                     # rows, blk, quad, 4
    e = np.where(rot[:, :, None, None] == 1, np.roll(e, -2, axis=3), e)    # position p <- (p+2)%4
    scale = (rs.astype(np.uint32) << 16).view(np.float32)
    bs = scale[:, None] * (2.0 ** s).astype(np.float32) * np.where(sign == 1, -1.0, 1.0).astype(np.float32)
    return (bs[:, :, None, None].astype(np.float32) * e).reshape(rows, cols).astype(np.float32)


def test_dequant_matches_reference_and_closed_form(orc, small, c1_codebook):
    cb = orc.unpack_codebook(c1_codebook)
    for case, (rows, cols) in (("a", (5, 64)), ("b", (16, 256)), ("c", (33, 512)), ("d", (8, 4096))):
        got = orc.dequantize(small[f"{case}_codes"], small[f"{case}_fields"], small[f"{case}_rs"],
                             rows, cols, cb)
        np.testing.assert_array_equal(got.view(np.uint32), small[f"{case}_deq"].view(np.uint32))
    got = orc.dequantize(small["rand_codes"], small["rand_fields"], small["rand_rs"], 16, 256, cb)
    np.testing.assert_array_equal(got.view(np.uint32), small["rand_deq"].view(np.uint32))
    closed = _numpy_dequant(small["rand_codes"], small["rand_fields"], small["rand_rs"], 16, 256, cb)
    np.testing.assert_array_equal(got.view(np.uint32), closed.view(np.uint32))


def test_gemv_matches_reference_and_dequant_dot(orc, small, c1_codebook):
    """expert_gemv_reference = (float) of the double dot of the dequantised row, bit for bit."""
    cb = orc.unpack_codebook(c1_codebook)
    for case, (rows, cols) in (("b", (16, 256)), ("d", (8, 4096))):
        x = small[f"{case}_x"]
        y = orc.gemv(small[f"{case}_codes"], small[f"{case}_fields"], small[f"{case}_rs"], rows, cols,
                     cb, x, 0.75)
        np.testing.assert_array_equal(y.view(np.uint32), small[f"{case}_gemv"].view(np.uint32))
        d = small[f"{case}_deq"].astype(np.float64)
        acc = np.zeros(rows)
        for r in range(rows):       # sequential double sum in column order
            s = 0.0
            for c in range(cols):
                s += float(d[r, c]) * float(x[c])
            acc[r] = s
        tmp = acc.astype(np.float32)
        np.testing.assert_array_equal(y, (np.float32(0.75) * tmp).astype(np.float32))
    x = small["rand_x"]
    y = orc.gemv(small["rand_codes"], small["rand_fields"], small["rand_rs"], 16, 256, cb, x, 1.0)
    np.testing.assert_array_equal(y.view(np.uint32), small["rand_gemv"].view(np.uint32))


def test_swiglu_matches_reference(orc, scalars):
    g, u = scalars["sw_g"], scalars["sw_u"]
    np.testing.assert_array_equal(orc.swiglu(g, u, 10.0).view(np.uint32), scalars["sw_out"].view(np.uint32))
    np.testing.assert_array_equal(orc.swiglu(g, u, 0.0).view(np.uint32),
                                  scalars["sw_out_nolimit"].view(np.uint32))
    # closed form: silu(min(g, 10)) * clamp(u, -10, 10)
    gg = np.minimum(g.astype(np.float64), 10.0)
    uu = np.clip(u.astype(np.float64), -10.0, 10.0)
    np.testing.assert_allclose(orc.swiglu(g, u, 10.0), gg / (1 + np.exp(-gg)) * uu, rtol=1e-5, atol=1e-6)


def test_route_softmax_topk(orc):
    rng = np.random.default_rng(6)
    lg = rng.standard_normal(256).astype(np.float32)
    lg[10] = lg[20] = 5.0                          # a tie: lower id first
    sel, w = orc.route(lg, 6)
    order = sorted(range(256), key=lambda e: (-lg[e], e))[:6]
    assert list(sel) == order and sel[0] == 10 and sel[1] == 20
    p = np.exp(lg[order].astype(np.float64) - lg.max())
    np.testing.assert_allclose(w, p / p.sum(), rtol=1e-6)
    assert abs(w.sum() - 1) < 1e-6


def test_route_topk_matches_reference(orc):
    """orc_route_topk (the engine router, src/engine/ops.cpp:62-92) against the reference's own
    outputs (tests/golden/route.npz: ties, the softplus guard, the sum floor, bias, top-6/8,
    renormalisation on and off, scaling 1 and 1.5), bit for bit; and the closed form of the
    score on a grid."""
    d = np.load(os.path.join(GOLDEN, "route.npz"))
    for i in range(d["logits"].shape[0]):
        k = int(d["k"][i])
        bias = d["bias"][i] if d["has_bias"][i] else None
        sel, w = orc.route_topk(d["logits"][i], bias, k, bool(d["norm"][i]), float(d["scaling"][i]))
        np.testing.assert_array_equal(sel, d["sel"][i][:k], err_msg=str(i))
        np.testing.assert_array_equal(w.view(np.uint32), d["w"][i][:k].view(np.uint32), err_msg=str(i))
    x = np.linspace(-30, 40, 701).astype(np.float32)
    got = np.array([orc.lib.orc_sqrtsoftplus(float(v)) for v in x], np.float32)
    ref = np.sqrt(np.where(x > 20, x.astype(np.float64), np.log1p(np.exp(x.astype(np.float64)))))
    np.testing.assert_allclose(got, ref, rtol=3e-7, atol=1e-30)


def test_route_topk_matches_live_reference(orc, ref):
    rng = np.random.default_rng(23)
    for i in range(200):
        lg = (rng.standard_normal(256) * rng.uniform(0.1, 8)).astype(np.float32)
        bias = rng.standard_normal(256).astype(np.float32) * 0.1 if i % 2 else None
        a = orc.route_topk(lg, bias, 6, True, 1.5)
        b = ref.route_topk(lg, bias, 6, True, 1.5)
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


# ---------------------------------------------------------------------------------------------
# the step after the routed experts: FP8 dense matvec, shared expert, hyper-connection post
# ---------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def step():
    return np.load(os.path.join(GOLDEN, "step.npz"))


def test_e8m0_matches_reference_and_closed_form(orc, step):
    got = np.array([orc.e8m0_to_float(i) for i in range(256)], np.float32)
    np.testing.assert_array_equal(got[:255].view(np.uint32), step["e8m0"][:255].view(np.uint32))
    assert np.isnan(got[255]) and np.isnan(step["e8m0"][255])
    np.testing.assert_array_equal(got[:255], np.ldexp(np.float32(1), np.arange(255) - 127).astype(np.float32))


def test_matvec_fp8_matches_reference_fixture(orc, step):
    """Bit for bit on the reference's outputs, ragged shapes included."""
    for i in range(3):
        y = orc.matvec_fp8(step[f"mv{i}_w"], step[f"mv{i}_s"], step[f"mv{i}_x"])
        np.testing.assert_array_equal(y.view(np.uint32), step[f"mv{i}_y"].view(np.uint32))


def test_matvec_fp8_matches_live_reference(orc, ref):
    rng = np.random.default_rng(8)
    for rows, cols in ((256, 4096), (2048, 1000), (1, 128)):
        w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] ^= 1
        s = rng.integers(100, 140, ((rows + 127) // 128, (cols + 127) // 128), dtype=np.uint8)
        x = rng.standard_normal(cols).astype(np.float32)
        np.testing.assert_array_equal(orc.matvec_fp8(w, s, x).view(np.uint32), ref.matvec_fp8(w, s, x).view(np.uint32))


def test_matvec_fp8_closed_forms(orc, scalars):
    """Against a float64 dense product of the decoded matrix (E4M3 table from the reference
    fixture, each 128x128 tile times 2^(s - 127)): a wrong tile index (row and column of the scale
    swapped, or the scale row not advancing every 128 rows) fails it. And an exact case: weights
    1.0 (0x38) times scale 2^3 against x = 1 gives 8 * cols."""
    rng = np.random.default_rng(9)
    rows, cols = 300, 640
    w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] ^= 1
    s = rng.integers(110, 130, (3, 5), dtype=np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    table = scalars["e4m3"].astype(np.float64)
    dense = table[w] * np.ldexp(1.0, np.repeat(np.repeat(s.astype(np.int64) - 127, 128, 0), 128, 1)[:rows, :cols])
    want = dense @ x.astype(np.float64)
    got = orc.matvec_fp8(w, s, x)
    assert np.max(np.abs(got - want) / (np.abs(dense) @ np.abs(x))) < 1e-5
    ones = np.full((rows, cols), 0x38, np.uint8)
    got = orc.matvec_fp8(ones, np.full((3, 5), 130, np.uint8), np.ones(cols, np.float32))
    np.testing.assert_array_equal(got, np.full(rows, 8.0 * cols, np.float32))


def test_shared_expert_composition(orc, scalars):
    """block += W_d . swiglu(W_g x, W_u x) against a float64 restatement from the decoded
    matrices; gate and up swapped, or the clamp dropped, fail it (the weights are scaled so that
    gate values pass the clamp limit)."""
    rng = np.random.default_rng(10)
    hidden, inter = 256, 384
    table = scalars["e4m3"].astype(np.float64)

    def mat(rows, cols, lo, hi):
        w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] ^= 1
        s = rng.integers(lo, hi, ((rows + 127) // 128, (cols + 127) // 128), dtype=np.uint8)
        d = table[w] * np.ldexp(1.0, np.repeat(np.repeat(s.astype(np.int64) - 127, 128, 0), 128, 1)[:rows, :cols])
        return w, s, d

    (wg, sg, dg), (wu, su, du), (wd, sd, dd) = mat(inter, hidden, 118, 121), mat(inter, hidden, 118, 121), \
        mat(hidden, inter, 112, 116)
    x = rng.standard_normal(hidden).astype(np.float32)
    block0 = rng.standard_normal(hidden).astype(np.float32)
    got = orc.shared_expert(wg, sg, wu, su, wd, sd, x, 10.0, block0.copy())
    g, u = dg @ x, du @ x
    assert (g > 10).any() and (np.abs(u) > 10).any()        # the clamp is exercised

    def swiglu(g, u, L):
        g = np.minimum(g, L)
        u = np.clip(u, -L, L)
        return g / (1 + np.exp(-g)) * u

    want = block0 + dd @ swiglu(g, u, 10.0)
    scale = np.abs(dd) @ np.abs(swiglu(g, u, 10.0)) + np.abs(block0)
    assert np.max(np.abs(got - want) / scale) < 1e-5
    for bad in (block0 + dd @ swiglu(u, g, 10.0), block0 + dd @ swiglu(g, u, 1e30)):
        assert np.max(np.abs(got - bad) / scale) > 1e-3


def test_hc_expand_matches_reference(orc, step):
    for nh in (1, 2, 4, 8):
        out = orc.hc_expand(step[f"hc{nh}_block"], step[f"hc{nh}_hc"], step[f"hc{nh}_post"], step[f"hc{nh}_comb"])
        np.testing.assert_array_equal(out.view(np.uint32), step[f"hc{nh}_out"].view(np.uint32))


def test_hc_expand_closed_form_and_add(orc):
    """Identity mixing (comb = I, post = 1) gives block + lane; a transposed comb index (dst * n_hc
    + src) fails the asymmetric case. hc_add is lane 0 + block."""
    rng = np.random.default_rng(11)
    nh, n = 4, 100
    hc = rng.standard_normal((nh, n)).astype(np.float32)
    blk = rng.standard_normal(n).astype(np.float32)
    out = orc.hc_expand(blk, hc, np.ones(nh, np.float32), np.eye(nh, dtype=np.float32).reshape(-1))
    np.testing.assert_array_equal(out, hc + blk)
    comb = np.arange(nh * nh, dtype=np.float32)
    out = orc.hc_expand(blk, hc, np.zeros(nh, np.float32), comb)
    want = np.stack([sum(comb[d + s * nh] * hc[s].astype(np.float64) for s in range(nh)) for d in range(nh)])
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)
    wrong = np.stack([sum(comb[d * nh + s] * hc[s].astype(np.float64) for s in range(nh)) for d in range(nh)])
    assert np.max(np.abs(out - wrong)) > 1.0
    np.testing.assert_array_equal(orc.hc_add(hc[0], blk), hc[0] + blk)


# ---- the reference's separable batch-pipeline steps ----------------------------------------------

def test_f32_to_e4m3_pinned(orc):
    """orc_f32_to_e4m3 against torch's float8_e4m3fn conversion (round to nearest even) on every
    code's value, every midpoint between neighbouring codes, points just off the midpoints and
    random values in +-448; a dropped tie rule or a wrong neighbour fails one of them."""
    torch = pytest.importorskip("torch")
    vals = np.array([orc.e4m3_to_float(c) for c in range(0x7F)], np.float32)
    mids = (vals[:-1] + vals[1:]) / 2
    off = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    rng = np.random.default_rng(6)
    rnd = (rng.random(4000) * 2 - 1).astype(np.float32) * rng.choice([448, 8, 1 / 64], 4000).astype(np.float32)
    x = np.concatenate([vals, mids, off, rnd]).astype(np.float32)
    x = np.concatenate([x, -x])
    got = np.array([orc.f32_to_e4m3(float(v)) for v in x], np.uint8)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, want)
    # ties really go to the even code (the midpoint above an odd code rounds up)
    assert orc.f32_to_e4m3(1.0625) == 0x38 and orc.f32_to_e4m3(1.1875) == 0x3A


def test_swiglu_quant_oracle_pinned(orc):
    """orc_swiglu_quant against the pinned orc_swiglu (the reference's SwiGLU, bit-identical to
    it) and orc_f32_to_e4m3: scale = max |v| / 448 per (slot, 128-row band), every byte the E4M3
    of v / scale, the band maximum at +-448; with the router weight, without it (w NULL = 1), and
    without the clamp (limit 0)."""
    rng = np.random.default_rng(8)
    dim, total = 256, 37
    g = rng.normal(0, 3, (dim, total)).astype(np.float32)
    u = rng.normal(0, 3, (dim, total)).astype(np.float32)
    g[:128, 5] = 0.0                               # an all-zero band: scale 1, bytes 0
    u[:128, 5] = 0.0
    gb = (g.view(np.uint32) >> 16).astype(np.uint16)   # truncated to bf16 bits (any bf16 will do)
    ub = (u.view(np.uint32) >> 16).astype(np.uint16)
    gf = (gb.astype(np.uint32) << 16).view(np.float32)
    uf = (ub.astype(np.uint32) << 16).view(np.float32)
    w = (0.1 + rng.random(total)).astype(np.float32)
    for wv, limit in ((w, 10.0), (None, 10.0), (w, 0.0)):
        out, sc = orc.swiglu_quant(gb, ub, wv, limit)
        a = np.zeros((dim, total), np.float32)
        for t in range(total):
            a[:, t] = orc.swiglu(np.ascontiguousarray(gf[:, t]), np.ascontiguousarray(uf[:, t]), limit)
        v = a * (np.float32(1) if wv is None else wv[None, :])
        for t in range(total):
            for kb in range(dim // 128):
                band = v[128 * kb:128 * kb + 128, t]
                m = np.float32(np.abs(band).max())
                want_sc = m * np.float32(1.0 / 448.0) if m > 0 else np.float32(1.0)
                assert sc[t, kb] == want_sc, (t, kb)
                inv = np.float32(1.0) / want_sc
                q = np.clip(band * inv, -448, 448).astype(np.float32)
                want = np.array([orc.f32_to_e4m3(float(e)) for e in q], np.uint8)
                np.testing.assert_array_equal(out[t, 128 * kb:128 * kb + 128], want)
                if m > 0:
                    assert (out[t, 128 * kb:128 * kb + 128] & 0x7F).max() == 0x7E
        assert (out[5, :128] == 0).all() and sc[5, 0] == 1.0


def test_scatter_slots_and_gather_tokens_oracle_brute_force(orc):
    """orc_scatter_slots and orc_gather_tokens against direct loops: the per-token sums in ord
    order from zero (float32, sequential), empty runs untouched; the gather a plain index copy."""
    rng = np.random.default_rng(9)
    dim, nb_tok, nb_stride = 24, 19, 32
    counts = rng.integers(0, 5, nb_tok)
    counts[3] = 0
    total = int(counts.sum())
    run = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    ordv = rng.permutation(total).astype(np.uint32)
    y = (rng.normal(0, 1, (dim, total)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    block0 = rng.normal(0, 1, (dim, nb_stride)).astype(np.float32)
    got = orc.scatter_slots(y, block0.copy(), ordv, run, nb_tok)
    want = block0.copy()
    yf = (y.astype(np.uint32) << 16).view(np.float32)
    for h in range(dim):
        for t in range(nb_tok):
            if run[t] == run[t + 1]:
                continue
            acc = np.float32(0)
            for i in range(run[t], run[t + 1]):
                acc = np.float32(acc + yf[h, ordv[i]])
            want[h, t] = np.float32(want[h, t] + acc)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    src = rng.normal(0, 1, (dim, nb_stride)).astype(np.float32)
    tok = rng.integers(0, nb_stride, 11).astype(np.uint32)
    np.testing.assert_array_equal(orc.gather_tokens(src, tok), src[:, tok])


def test_expert_gemm_w8a8_oracle_pinned(orc, c1_codebook):
    """orc_expert_gemm_w8a8 against numpy built on the closed-form dequant above (row scale 1
    gives each weight's E4M3 value): each 128-column block's sum in float64, the fold over blocks
    as an f32 fma in block order (a product of two f32 is exact in float64), the row scale times
    wscale last. Token ids with a repeat, a strided output (the other columns untouched) and the
    bf16 output (round to nearest even of the f32 result). The per-block activation scales differ
    by block, so a block mix-up or a fold out of order fails."""
    rng = np.random.default_rng(21)
    rows, cols, ntok = 32, 1024, 10
    nkb = cols // 128
    cb = orc.unpack_codebook(c1_codebook)
    codes = rng.integers(0, 256, rows * cols * 10 // 32, dtype=np.uint8)
    fields = rng.integers(0, 256, rows * cols * 6 // 128, dtype=np.uint8)
    rs = (rng.uniform(4e-4, 2e-3, rows).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    w8 = _numpy_dequant(codes, fields, np.full(rows, 0x3F80, np.uint16), rows, cols, cb).astype(np.float64)
    x8 = rng.integers(0, 256, (ntok, cols), dtype=np.uint8)
    x8[(x8 & 0x7F) == 0x7F] ^= 1                       # no NaN codes
    e4 = np.array([orc.e4m3_to_float(b) for b in range(256)], np.float64)
    xs = rng.uniform(0.01, 2.0, (ntok, nkb)).astype(np.float32)
    tok = np.array([3, 0, 9, 4, 4, 7, 1], np.uint32)
    nt, wscale = len(tok), 0.75
    rsw = (rs.astype(np.uint32) << 16).view(np.float32) * np.float32(wscale)
    want = np.zeros((rows, nt), np.float32)
    for j, t in enumerate(tok):
        raw = (w8.reshape(rows, nkb, 128) * e4[x8[t]].reshape(1, nkb, 128)).sum(axis=2).astype(np.float32)
        out = np.zeros(rows, np.float32)
        for kb in range(nkb):
            out = (raw[:, kb].astype(np.float64) * np.float64(xs[t, kb]) + out.astype(np.float64)).astype(np.float32)
        want[:, j] = out * rsw
    got = orc.expert_gemm_w8a8(codes, fields, rs, tok, nt, x8, xs, cb, rows, cols, wscale)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=0)
    # strided into an existing output: columns past nt keep their values
    y = np.full((rows, 9), 7.0, np.float32)
    got9 = orc.expert_gemm_w8a8(codes, fields, rs, tok, nt, x8, xs, cb, rows, cols, wscale, ld=9, y=y)
    np.testing.assert_array_equal(got9[:, :nt].view(np.uint32), got.view(np.uint32))
    assert (got9[:, nt:] == 7.0).all()
    # bf16: the f32 result rounded to nearest even; identity token ids
    gb = orc.expert_gemm_w8a8(codes, fields, rs, None, 5, x8, xs, cb, rows, cols, wscale, y_bf16=True)
    gf = orc.expert_gemm_w8a8(codes, fields, rs, None, 5, x8, xs, cb, rows, cols, wscale)
    u = gf.view(np.uint32).astype(np.uint64)
    np.testing.assert_array_equal(gb, ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16))
