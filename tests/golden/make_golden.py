"""Writes the golden fixtures under tests/golden/ from the reference's own CPU path.

Run in the build container (the only place the reference tree exists):

    make -C oracle && python tests/golden/make_golden.py

The reference functions run from oracle/_ref/libaffref.so, which oracle/Makefile compiles from
the reference sources where they lie (blockquant.cpp, aff_format.cpp, source_dtypes.cpp,
expert_kernel.cpp, threadpool.cpp, ops.cpp, log.cpp) plus a C-ABI forwarder. Inputs come from
the synthetic generator (splitmix64 + Box-Muller, bf16 RNE; seeds fixed by the benchmark
configs); the generator itself is pinned separately by tests/test_oracle.py.

Fixtures (data only: inputs and the reference's outputs):
  c1_codebook.bin   uint32[2048]  packed E4M3 quad codebook fitted on the config-1 expert
                                  (samples 2^19 per matrix, fit_codebook(50, seed 1), projection)
  c1_manifest.json  SHA-256 of the config-1 inputs, of the nine quantised planes, of the
                    dequantised matrices and of the FFN intermediates; sampled plane rows
  c1_ffn_y.bin      float32[4096] FFN output y = W_d . swiglu(W_g x, W_u x) (weight 1)
  small.npz         small matrices (edge rows, importance, odd shapes) with the reference's
                    planes, dequantised values and GEMV outputs
  scalars.npz       E4M3 table, bf16 rounding cases, swiglu cases
  route.npz         the engine router (route_topk): logits and bias cases with the chosen
                    experts and weights
  fit_large.npz     a codebook fit at aff-quantize's scale: 8 matrices (seeds 3000-3007, 2048x4096
                    and 4096x2048 alternating, bf16 0.02 N(0,1)), 2^19 samples each, the raw
                    fit_codebook(50, seed 1) (written by `make_golden.py fit_large`)
  step.npz          the step after the routed experts: FP8 dense matvecs (matvec_dense over E4M3
                    weights with UE8M0 128x128 tile scales, ragged shapes included), the E8M0
                    table, and hc_expand cases for n_hc 1, 2, 4, 8
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import load_oracle, load_ref  # noqa: E402
from oracle.binding import H, I  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
S_W, S_X = 1000, 7


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_inputs(O):
    wg = O.normal_bf16(S_W + 0, I * H, 0.02).reshape(I, H)
    wu = O.normal_bf16(S_W + 1, I * H, 0.02).reshape(I, H)
    wd = O.normal_bf16(S_W + 2, H * I, 0.02).reshape(H, I)
    x = O.normal_bf16(S_X, H, 1.0)
    return wg, wu, wd, x


def row_slices(planes, rows, cols, pick):
    """hex of selected rows of each plane (codes, fields, rscales)."""
    codes, fields, rs = planes
    cb_row, f_row = cols * 10 // 32, cols * 6 // 128
    out = {}
    for r in pick:
        out[str(r)] = {
            "codes": codes[r * cb_row:(r + 1) * cb_row].tobytes().hex(),
            "fields": fields[r * f_row:(r + 1) * f_row].tobytes().hex(),
            "rscale": int(rs[r]),
        }
    return out


def make_c1(O, R):
    t0 = time.time()
    wg, wu, wd, x = c1_inputs(O)
    samples = np.concatenate([R.collect_samples(w, 1 << 19) for w in (wg, wu, wd)])
    print(f"samples: {samples.size} floats", flush=True)
    cb = R.fit_codebook(samples, 50, 1, project=True)
    packed = R.pack_codebook(cb)
    assert np.array_equal(R.unpack_codebook(packed).view(np.uint32), cb.view(np.uint32))
    packed.astype("<u4").tofile(os.path.join(OUT, "c1_codebook.bin"))
    print(f"codebook fitted in {time.time() - t0:.0f} s", flush=True)

    man = {"seeds": {"S_W": S_W, "S_X": S_X, "fit_seed": 1, "fit_iters": 50, "budget": 1 << 19},
           "inputs": {"gate": sha(wg), "up": sha(wu), "down": sha(wd), "x": sha(x)},
           "codebook_f32": sha(cb), "planes": {}, "dequant": {}, "rows": {}}
    mats = {"gate": (wg, I, H), "up": (wu, I, H), "down": (wd, H, I)}
    deq = {}
    qs = {}
    for name, (w, rows, cols) in mats.items():
        t = time.time()
        q = R.quantize(w, cb, None, search=True)
        qs[name] = q
        man["planes"][name] = {"codes": sha(q[0]), "fields": sha(q[1]), "rscales": sha(q[2])}
        man["rows"][name] = row_slices(q, rows, cols, [0, 1, rows // 2 + 3, rows - 1])
        d = R.dequantize(*q, rows, cols, cb)
        deq[name] = d
        man["dequant"][name] = sha(d)
        print(f"{name}: quantised in {time.time() - t:.0f} s", flush=True)
    # importance = all ones gives the same bytes as none (the config-1 "uniform importance")
    ones = np.ones(H, np.float32)
    qi = R.quantize(wg[:64].copy(), cb, ones, search=True)
    man["gate64_ones_importance_equals_none"] = bool(
        sha(qi[0]) == sha(qs["gate"][0][: 64 * H * 10 // 32]) and sha(qi[1]) == sha(qs["gate"][1][: 64 * H * 6 // 128]))

    g = R.gemv(*qs["gate"], I, H, cb, x)
    u = R.gemv(*qs["up"], I, H, cb, x)
    a = R.swiglu(g, u, 10.0)
    y = R.gemv(*qs["down"], H, I, cb, a, 1.0)
    man["ffn"] = {"g": sha(g), "u": sha(u), "a": sha(a), "y": sha(y)}
    y.astype("<f4").tofile(os.path.join(OUT, "c1_ffn_y.bin"))
    with open(os.path.join(OUT, "c1_manifest.json"), "w") as f:
        json.dump(man, f, indent=1, sort_keys=True)
    print(f"config 1 done in {time.time() - t0:.0f} s", flush=True)
    return cb


def make_small(O, R, cb):
    rng = np.random.default_rng(20261201)
    cases = {}
    # shapes: the smallest legal row (64 cols keeps rows byte-aligned), ragged row counts
    for name, rows, cols in (("a", 5, 64), ("b", 16, 256), ("c", 33, 512), ("d", 8, 4096)):
        w = O.normal_bf16(5000 + rows * 7 + cols, rows * cols, 0.02).reshape(rows, cols).copy()
        if rows >= 5:
            w[1] = 0.0                                    # an all-zero row
            w[2, 16:32] = 0.0                             # an all-zero block
            w[3, 5] = 3.0                                 # one outlier dominates the row scale
            w[4] *= -1.0
        imp = rng.uniform(0.1, 4.0, cols).astype(np.float32)
        q = R.quantize(w, cb, None, search=True)
        qn = R.quantize(w, cb, None, search=False)
        qi = R.quantize(w, cb, imp, search=True)
        x = O.normal_bf16(6000 + cols, cols, 1.0)
        d = R.dequantize(*q, rows, cols, cb)
        y = R.gemv(*q, rows, cols, cb, x, 0.75)
        cases.update({f"{name}_w": w, f"{name}_imp": imp, f"{name}_x": x,
                      f"{name}_codes": q[0], f"{name}_fields": q[1], f"{name}_rs": q[2],
                      f"{name}_codes_nosearch": qn[0], f"{name}_fields_nosearch": qn[1],
                      f"{name}_codes_imp": qi[0], f"{name}_fields_imp": qi[1],
                      f"{name}_deq": d, f"{name}_gemv": y})
    # arbitrary planes (every field value, random codes) dequantised by the reference
    rows, cols = 16, 256
    codes = rng.integers(0, 256, rows * cols * 10 // 32, dtype=np.uint8)
    fields = rng.integers(0, 256, rows * cols * 6 // 128, dtype=np.uint8)
    rs = np.array([R.float_to_bf16(v) for v in rng.uniform(1e-4, 1e-1, rows).astype(np.float32)], np.uint16)
    cases["rand_codes"], cases["rand_fields"], cases["rand_rs"] = codes, fields, rs
    cases["rand_deq"] = R.dequantize(codes, fields, rs, rows, cols, cb)
    xr = O.normal_bf16(6100, cols, 1.0)
    cases["rand_x"] = xr
    cases["rand_gemv"] = R.gemv(codes, fields, rs, rows, cols, cb, xr, 1.0)
    # a small codebook fit (trajectory check at a size the CPU suite can rerun)
    w = O.normal_bf16(7000, 256 * 1024, 0.02).reshape(256, 1024)
    s = R.collect_samples(w, 1 << 16)
    cases["fit_samples"] = s
    cases["fit_cb_raw"] = R.fit_codebook(s, 50, 1, project=False)
    cases["fit_cb_proj"] = R.fit_codebook(s, 50, 1, project=True)
    np.savez_compressed(os.path.join(OUT, "small.npz"), **cases)


def make_fit_large(O, R):
    t0 = time.time()
    parts = []
    for i in range(8):
        rows, cols = (I, H) if i % 2 == 0 else (H, I)
        w = O.normal_bf16(3000 + i, rows * cols, 0.02).reshape(rows, cols)
        parts.append(R.collect_samples(w, 1 << 19))
    s = np.concatenate(parts)
    print(f"fit_large: {s.size} samples", flush=True)
    cb = R.fit_codebook(s, 50, 1, project=False)
    np.savez_compressed(os.path.join(OUT, "fit_large.npz"), cb_raw=cb, n_samples=np.array(s.size),
                        samples_sha256=np.array(sha(s)))
    print(f"fit_large done in {time.time() - t0:.0f} s", flush=True)


def make_scalars(O, R):
    e4 = np.array([R.e4m3_to_float(b) for b in range(256)], np.float32)
    rng = np.random.default_rng(7)
    f = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 1.01171875, 3.3895314e38,
                                  1e-40, -1e-40, 65504.0], np.float32)]).astype(np.float32)
    bf = np.array([R.float_to_bf16(v) for v in f], np.uint16)
    g = np.concatenate([np.linspace(-30, 30, 601, dtype=np.float32), rng.standard_normal(500).astype(np.float32) * 5])
    u = np.concatenate([np.linspace(30, -30, 601, dtype=np.float32), rng.standard_normal(500).astype(np.float32) * 5])
    sw = R.swiglu(g, u, 10.0)
    sw0 = R.swiglu(g, u, 0.0)
    np.savez_compressed(os.path.join(OUT, "scalars.npz"), e4m3=e4, bf_in=f, bf_out=bf, sw_g=g, sw_u=u,
                        sw_out=sw, sw_out_nolimit=sw0)


def make_route(R):
    """route_topk cases: N(0,1) logits with and without a bias, exact ties (lower id wins), logits
    past softplus's x > 20 guard, very negative logits (the sum floor), top-6 and top-8, with and
    without renormalisation, scaling 1 and 1.5."""
    rng = np.random.default_rng(17)
    E = 256
    cases = []
    for i in range(40):
        lg = rng.standard_normal(E).astype(np.float32) * (1.0 if i % 4 else 3.0)
        bias = (rng.standard_normal(E).astype(np.float32) * 0.05) if i % 2 else None
        if i % 5 == 0:
            lg[rng.choice(E, 8, replace=False)] = lg.max() + 0.5          # an 8-way tie at the top
        if i % 7 == 0:
            lg[rng.choice(E, 3, replace=False)] = 25.0 + i                # past the x > 20 guard
        if i == 39:
            lg[:] = -60.0                                                  # sum below the fp16 floor
        k = 8 if i % 3 == 0 else 6
        norm = i % 6 != 5
        scaling = 1.5 if i % 2 else 1.0
        sel, w = R.route_topk(lg, bias, k, norm, scaling)
        cases.append((lg, np.zeros(E, np.float32) if bias is None else bias, bias is not None, k, norm, scaling,
                      np.pad(sel, (0, 8 - sel.size)), np.pad(w, (0, 8 - w.size))))
    np.savez_compressed(os.path.join(OUT, "route.npz"),
                        logits=np.stack([c[0] for c in cases]), bias=np.stack([c[1] for c in cases]),
                        has_bias=np.array([c[2] for c in cases]), k=np.array([c[3] for c in cases], np.uint32),
                        norm=np.array([c[4] for c in cases]), scaling=np.array([c[5] for c in cases], np.float32),
                        sel=np.stack([c[6] for c in cases]).astype(np.uint32),
                        w=np.stack([c[7] for c in cases]).astype(np.float32))


def make_step(R):
    """matvec_fp8 (src/engine/matvec_fp8.inc:42-82) on three shapes, one ragged in both directions,
    with every E4M3 code but the NaNs and scales 2^-16 .. 2^8; e8m0_to_float for every byte;
    hc_expand (src/engine/ops.cpp:470-482) for each n_hc."""
    rng = np.random.default_rng(23)
    out = {"e8m0": np.array([R.e8m0_to_float(i) for i in range(256)], np.float32)}
    for i, (rows, cols) in enumerate(((128, 256), (200, 300), (129, 512))):
        w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] ^= 1
        s = rng.integers(111, 136, ((rows + 127) // 128, (cols + 127) // 128), dtype=np.uint8)
        x = rng.standard_normal(cols).astype(np.float32)
        out[f"mv{i}_w"], out[f"mv{i}_s"], out[f"mv{i}_x"] = w, s, x
        out[f"mv{i}_y"] = R.matvec_fp8(w, s, x)
    for nh in (1, 2, 4, 8):
        n = 300
        hc = rng.standard_normal((nh, n)).astype(np.float32)
        blk = rng.standard_normal(n).astype(np.float32)
        post = rng.standard_normal(nh).astype(np.float32)
        comb = rng.standard_normal(nh * nh).astype(np.float32)
        out[f"hc{nh}_hc"], out[f"hc{nh}_block"], out[f"hc{nh}_post"], out[f"hc{nh}_comb"] = hc, blk, post, comb
        out[f"hc{nh}_out"] = R.hc_expand(blk, hc, post, comb)
    np.savez_compressed(os.path.join(OUT, "step.npz"), **out)


def main():
    O, R = load_oracle(), load_ref()
    make_route(R)
    make_step(R)
    make_scalars(O, R)
    cb = make_c1(O, R)
    make_small(O, R, cb)
    print("fixtures written to", OUT)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "fit_large":  # only the large-fit fixture
        make_fit_large(load_oracle(), load_ref())
    elif len(sys.argv) > 1 and sys.argv[1] == "route":     # only the router fixture
        make_route(load_ref())
    elif len(sys.argv) > 1 and sys.argv[1] == "step":    # only the step-after fixture
        make_step(load_ref())
    else:
        main()
