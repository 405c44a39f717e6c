"""numpy-facing ctypes bindings for the oracle and the reference build (test infrastructure)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libaffref.so")
REF_TREE = "/root/reference"

H, I = 4096, 2048          # V4-Flash hidden size and routed-expert intermediate size
N_CB = 2 * 1024 * 4         # floats in a codebook [variant][code][4]

_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be C-contiguous"
    return a.ctypes.data_as(t)


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so (always) and _ref/libaffref.so (when the reference tree exists)."""
    targets = ["oracle"]
    if ref is None:
        ref = os.path.isdir(REF_TREE)
    if ref:
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def plane_bytes(rows: int, cols: int) -> tuple[int, int, int]:
    """(code bytes, field bytes, rscale bytes) of one [rows x cols] matrix."""
    return rows * cols * 10 // 32, rows * cols * 6 // 128, rows * 2


class Oracle:
    """The C restatement (oracle/oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.orc_set_threads.argtypes = [C.c_int]
        L.orc_get_threads.restype = C.c_int
        L.orc_e4m3_to_float.argtypes = [C.c_uint8]
        L.orc_e4m3_to_float.restype = C.c_float
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_pack_bits.argtypes = [_u8p, C.c_uint64, C.c_uint32, C.c_uint32]
        L.orc_unpack_bits.argtypes = [_u8p, C.c_uint64, C.c_uint32]
        L.orc_unpack_bits.restype = C.c_uint32
        L.orc_splitmix_at.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_splitmix_at.restype = C.c_uint64
        L.orc_gen_normal_bf16.argtypes = [C.c_uint64, C.c_uint64, C.c_double, _f32p]
        L.orc_gen_normal_f64.argtypes = [C.c_uint64, C.c_uint64, _f64p]
        L.orc_expert_layout.argtypes = [C.c_uint64, C.c_uint64, _u64p, _u64p]
        L.orc_expert_layout.restype = C.c_uint64
        L.orc_collect_samples.argtypes = [_f32p, C.c_uint64, C.c_uint64, C.c_uint64, _f32p, C.c_uint64]
        L.orc_collect_samples.restype = C.c_uint64
        L.orc_fit_codebook.argtypes = [_f32p, C.c_uint64, C.c_uint32, C.c_uint64, _f32p]
        L.orc_e4m3_nearest.argtypes = [C.c_float]
        L.orc_e4m3_nearest.restype = C.c_uint8
        L.orc_project_codebook.argtypes = [_f32p, C.c_uint64]
        L.orc_pack_codebook.argtypes = [_f32p, _u32p]
        L.orc_unpack_codebook.argtypes = [_u32p, _f32p]
        L.orc_codebook_exponents_ok.argtypes = [_u32p]
        L.orc_codebook_exponents_ok.restype = C.c_int
        L.orc_quantize_matrix.argtypes = [_f32p, C.c_uint64, C.c_uint64, _f32p, _f32p, _u8p, _u8p, _u16p]
        L.orc_quantize_matrix.restype = C.c_int
        L.orc_dequantize_matrix.argtypes = [_u8p, _u8p, _u16p, C.c_uint64, C.c_uint64, _f32p, _f32p]
        L.orc_dequantize_matrix.restype = C.c_int
        L.orc_expert_gemv.argtypes = [_u8p, _u8p, _u16p, C.c_uint64, C.c_uint64, _f32p, _f32p, C.c_float, _f32p]
        L.orc_swiglu.argtypes = [_f32p, _f32p, C.c_uint64, C.c_float, _f32p]
        L.orc_expert_ffn.argtypes = [_u8p, C.c_uint64, C.c_uint64, _f32p, _f32p, C.c_float, C.c_float, _f32p]
        L.orc_route_softmax_topk.argtypes = [_f32p, C.c_uint32, C.c_uint32, _u32p, _f32p]
        L.orc_sqrtsoftplus.argtypes = [C.c_float]
        L.orc_sqrtsoftplus.restype = C.c_float
        L.orc_route_topk.argtypes = [_f32p, _f32p, C.c_uint32, C.c_uint32, C.c_int, C.c_float, _u32p, _f32p]
        L.orc_route_topk.restype = C.c_uint32
        L.orc_e8m0_to_float.argtypes = [C.c_uint8]
        L.orc_e8m0_to_float.restype = C.c_float
        L.orc_matvec_fp8.argtypes = [_u8p, _u8p, C.c_uint64, C.c_uint64, _f32p, _f32p]
        L.orc_shared_expert.argtypes = [_u8p, _u8p, _u8p, _u8p, _u8p, _u8p, C.c_uint64, C.c_uint64, C.c_float,
                                        _f32p, _f32p]
        L.orc_hc_expand.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_uint32, C.c_uint32]
        L.orc_hc_add.argtypes = [_f32p, _f32p, C.c_uint32]
        L.orc_f32_to_e4m3.argtypes = [C.c_float]
        L.orc_f32_to_e4m3.restype = C.c_uint8
        L.orc_swiglu_quant.argtypes = [_u16p, _u16p, _f32p, _u8p, _f32p, C.c_uint32, C.c_uint32, C.c_float]
        L.orc_scatter_slots.argtypes = [_u16p, _f32p, _u32p, _u32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_gather_tokens.argtypes = [_f32p, _f32p, _u32p, C.c_uint32, C.c_uint32, C.c_uint32]
        L.orc_expert_gemm_w8a8.argtypes = [_u8p, _u8p, _u16p, _u32p, C.c_uint32, C.c_uint32, _u8p, _f32p, _f32p,
                                           C.c_uint64, C.c_uint64, C.c_float, C.c_int, C.c_void_p]

    # -- threads ---------------------------------------------------------------------------
    def set_threads(self, n: int) -> None:
        self.lib.orc_set_threads(int(n))

    def threads(self) -> int:
        return int(self.lib.orc_get_threads())

    # -- codecs ----------------------------------------------------------------------------
    def e4m3_to_float(self, b: int) -> float:
        return float(self.lib.orc_e4m3_to_float(b))

    def f32_to_bf16(self, f: float) -> int:
        return int(self.lib.orc_f32_to_bf16(f))

    def f32_to_e4m3(self, f: float) -> int:
        return int(self.lib.orc_f32_to_e4m3(f))

    # -- the reference's separable batch-pipeline steps ----------------------------------------
    def swiglu_quant(self, g: np.ndarray, u: np.ndarray, w, limit: float):
        """g, u: uint16 (bf16 bits) [dim][total]; w f32 [total] or None -> (out u8 [total][dim],
        scales f32 [total][dim/128])."""
        dim, total = g.shape
        out = np.zeros((total, dim), np.uint8)
        scales = np.zeros((total, dim // 128), np.float32)
        wp = None if w is None else _p(np.ascontiguousarray(w, np.float32), _f32p)
        self.lib.orc_swiglu_quant(_p(np.ascontiguousarray(g, np.uint16), _u16p), _p(np.ascontiguousarray(u, np.uint16), _u16p),
                                  wp, _p(out, _u8p), _p(scales, _f32p), dim, total, float(limit))
        return out, scales

    def scatter_slots(self, y: np.ndarray, block: np.ndarray, ord_: np.ndarray, run: np.ndarray, nb_tok: int):
        dim, total = y.shape
        self.lib.orc_scatter_slots(_p(np.ascontiguousarray(y, np.uint16), _u16p), _p(block, _f32p),
                                   _p(np.ascontiguousarray(ord_, np.uint32), _u32p),
                                   _p(np.ascontiguousarray(run, np.uint32), _u32p), dim, nb_tok, block.shape[1], total)
        return block

    def gather_tokens(self, src: np.ndarray, tok: np.ndarray) -> np.ndarray:
        dim, nb = src.shape
        nt = tok.size
        dst = np.zeros((dim, nt), np.float32)
        self.lib.orc_gather_tokens(_p(np.ascontiguousarray(src, np.float32), _f32p), _p(dst, _f32p),
                                   _p(np.ascontiguousarray(tok, np.uint32), _u32p), dim, nb, nt)
        return dst

    def expert_gemm_w8a8(self, codes: np.ndarray, fields: np.ndarray, rscales: np.ndarray, tok, nt: int,
                         x8: np.ndarray, xs: np.ndarray, cb: np.ndarray, rows: int, cols: int, wscale: float,
                         y_bf16: bool = False, ld: int = 0, y: np.ndarray | None = None) -> np.ndarray:
        """One tile of the W8A8 GEMM: planes in container layout (one matrix), tok uint32 [nt] or
        None, x8 uint8 [tokens][cols], xs f32 [tokens][cols/128] -> y [rows][ld or nt] (f32, or
        uint16 bf16 bits); an existing y keeps its other columns."""
        yld = ld if ld else nt
        if y is None:
            y = np.zeros((rows, yld), np.uint16 if y_bf16 else np.float32)
        tp = None if tok is None else _p(np.ascontiguousarray(tok, np.uint32), _u32p)
        self.lib.orc_expert_gemm_w8a8(_p(np.ascontiguousarray(codes, np.uint8), _u8p),
                                      _p(np.ascontiguousarray(fields, np.uint8), _u8p),
                                      _p(np.ascontiguousarray(rscales).view(np.uint16), _u16p), tp, nt, ld,
                                      _p(np.ascontiguousarray(x8, np.uint8), _u8p),
                                      _p(np.ascontiguousarray(xs, np.float32), _f32p),
                                      _p(np.ascontiguousarray(cb, np.float32), _f32p), rows, cols, float(wscale),
                                      int(bool(y_bf16)), y.ctypes.data)
        return y

    def e4m3_nearest(self, f: float) -> int:
        return int(self.lib.orc_e4m3_nearest(f))

    # -- generator -------------------------------------------------------------------------
    def splitmix_at(self, seed: int, k: int) -> int:
        return int(self.lib.orc_splitmix_at(seed, k))

    def normal_bf16(self, seed: int, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.lib.orc_gen_normal_bf16(seed, n, scale, _p(out, _f32p))
        return out

    def normal_f64(self, seed: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float64)
        self.lib.orc_gen_normal_f64(seed, n, _p(out, _f64p))
        return out

    # -- geometry --------------------------------------------------------------------------
    def expert_layout(self, hidden: int = H, inter: int = I):
        off = np.zeros(9, np.uint64)
        size = np.zeros(9, np.uint64)
        stride = self.lib.orc_expert_layout(hidden, inter, _p(off, _u64p), _p(size, _u64p))
        return int(stride), off.astype(np.int64), size.astype(np.int64)

    # -- codebook --------------------------------------------------------------------------
    def collect_samples(self, w: np.ndarray, budget: int) -> np.ndarray:
        rows, cols = w.shape
        n = self.lib.orc_collect_samples(_p(w, _f32p), rows, cols, budget, None, 0)
        out = np.empty(n, np.float32)
        self.lib.orc_collect_samples(_p(w, _f32p), rows, cols, budget, _p(out, _f32p), n)
        return out

    def fit_codebook(self, samples: np.ndarray, iters: int = 50, seed: int = 1) -> np.ndarray:
        cb = np.zeros(N_CB, np.float32)
        self.lib.orc_fit_codebook(_p(samples, _f32p), samples.size, iters, seed, _p(cb, _f32p))
        return cb

    def project_codebook(self, cb: np.ndarray) -> np.ndarray:
        out = np.ascontiguousarray(cb, np.float32).copy()
        self.lib.orc_project_codebook(_p(out, _f32p), out.size)
        return out

    def pack_codebook(self, cb: np.ndarray) -> np.ndarray:
        out = np.zeros(2048, np.uint32)
        self.lib.orc_pack_codebook(_p(np.ascontiguousarray(cb, np.float32), _f32p), _p(out, _u32p))
        return out

    def unpack_codebook(self, packed: np.ndarray) -> np.ndarray:
        out = np.zeros(N_CB, np.float32)
        self.lib.orc_unpack_codebook(_p(np.ascontiguousarray(packed, np.uint32), _u32p), _p(out, _f32p))
        return out

    def codebook_exponents_ok(self, packed: np.ndarray) -> bool:
        return bool(self.lib.orc_codebook_exponents_ok(_p(np.ascontiguousarray(packed, np.uint32), _u32p)))

    # -- quantise / dequantise ---------------------------------------------------------------
    def quantize(self, w: np.ndarray, cb: np.ndarray, importance: np.ndarray | None = None):
        rows, cols = w.shape
        nc, nf, _ = plane_bytes(rows, cols)
        codes = np.zeros(nc, np.uint8)
        fields = np.zeros(nf, np.uint8)
        rs = np.zeros(rows, np.uint16)
        imp = None if importance is None else _p(np.ascontiguousarray(importance, np.float32), _f32p)
        rc = self.lib.orc_quantize_matrix(_p(np.ascontiguousarray(w, np.float32), _f32p), rows, cols,
                                          _p(cb, _f32p), imp, _p(codes, _u8p), _p(fields, _u8p),
                                          _p(rs, _u16p))
        if rc != 0:
            raise ValueError("orc_quantize_matrix refused the shape")
        return codes, fields, rs

    def dequantize(self, codes, fields, rs, rows: int, cols: int, cb: np.ndarray) -> np.ndarray:
        out = np.empty((rows, cols), np.float32)
        rc = self.lib.orc_dequantize_matrix(_p(codes, _u8p), _p(fields, _u8p), _p(rs, _u16p), rows,
                                            cols, _p(cb, _f32p), _p(out, _f32p))
        if rc != 0:
            raise ValueError("orc_dequantize_matrix refused the shape")
        return out

    def gemv(self, codes, fields, rs, rows, cols, cb, x, w=1.0, y=None) -> np.ndarray:
        y = np.zeros(rows, np.float32) if y is None else y
        self.lib.orc_expert_gemv(_p(codes, _u8p), _p(fields, _u8p), _p(rs, _u16p), rows, cols,
                                 _p(cb, _f32p), _p(np.ascontiguousarray(x, np.float32), _f32p),
                                 float(w), _p(y, _f32p))
        return y

    def swiglu(self, g: np.ndarray, u: np.ndarray, limit: float = 10.0) -> np.ndarray:
        out = np.empty_like(g, dtype=np.float32)
        self.lib.orc_swiglu(_p(g, _f32p), _p(u, _f32p), g.size, limit, _p(out, _f32p))
        return out

    def expert_ffn(self, expert: np.ndarray, cb: np.ndarray, x: np.ndarray, w: float = 1.0,
                   limit: float = 10.0, y: np.ndarray | None = None, hidden: int = H,
                   inter: int = I) -> np.ndarray:
        y = np.zeros(hidden, np.float32) if y is None else y
        self.lib.orc_expert_ffn(_p(expert, _u8p), hidden, inter, _p(cb, _f32p),
                                _p(np.ascontiguousarray(x, np.float32), _f32p), float(w), limit,
                                _p(y, _f32p))
        return y

    def route_topk(self, logits: np.ndarray, bias: np.ndarray | None, k: int = 6, norm: bool = True,
                   scaling: float = 1.0):
        """The engine's router (sqrtsoftplus + bias for selection, renormalised, scaled)."""
        sel = np.zeros(k, np.uint32)
        w = np.zeros(k, np.float32)
        lg = np.ascontiguousarray(logits, np.float32)
        b = None if bias is None else _p(np.ascontiguousarray(bias, np.float32), _f32p)
        n = self.lib.orc_route_topk(_p(lg, _f32p), b, lg.size, k, int(norm), scaling, _p(sel, _u32p), _p(w, _f32p))
        return sel[:n], w[:n]

    def route(self, logits: np.ndarray, k: int = 6):
        sel = np.zeros(k, np.uint32)
        w = np.zeros(k, np.float32)
        lg = np.ascontiguousarray(logits, np.float32)
        self.lib.orc_route_softmax_topk(_p(lg, _f32p), lg.size, k, _p(sel, _u32p), _p(w, _f32p))
        return sel, w

    # -- shared expert and hyper-connection post -----------------------------------------------
    def e8m0_to_float(self, b: int) -> float:
        return float(self.lib.orc_e8m0_to_float(b))

    def matvec_fp8(self, w: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
        """w [rows x cols] E4M3 bytes, s [ceil(rows/128) x ceil(cols/128)] UE8M0 bytes."""
        rows, cols = w.shape
        out = np.zeros(rows, np.float32)
        self.lib.orc_matvec_fp8(_p(w, _u8p), _p(s, _u8p), rows, cols,
                                _p(np.ascontiguousarray(x, np.float32), _f32p), _p(out, _f32p))
        return out

    def shared_expert(self, wg, sg, wu, su, wd, sd, x: np.ndarray, limit: float = 10.0,
                      block: np.ndarray | None = None) -> np.ndarray:
        """block += W_d . swiglu(W_g x, W_u x) for one token (FP8 dense weights)."""
        inter, hidden = wg.shape
        block = np.zeros(hidden, np.float32) if block is None else block
        self.lib.orc_shared_expert(_p(wg, _u8p), _p(sg, _u8p), _p(wu, _u8p), _p(su, _u8p), _p(wd, _u8p),
                                   _p(sd, _u8p), hidden, inter, limit,
                                   _p(np.ascontiguousarray(x, np.float32), _f32p), _p(block, _f32p))
        return block

    def hc_expand(self, block: np.ndarray, hc: np.ndarray, post: np.ndarray, comb: np.ndarray) -> np.ndarray:
        """hc [n_hc x n_embd], post [n_hc], comb [n_hc * n_hc] -> next state [n_hc x n_embd]."""
        n_hc, n = hc.shape
        out = np.zeros((n_hc, n), np.float32)
        self.lib.orc_hc_expand(_p(out, _f32p), _p(np.ascontiguousarray(block, np.float32), _f32p),
                               _p(np.ascontiguousarray(hc, np.float32), _f32p),
                               _p(np.ascontiguousarray(post, np.float32), _f32p),
                               _p(np.ascontiguousarray(comb, np.float32), _f32p), n, n_hc)
        return out

    def hc_add(self, hc: np.ndarray, block: np.ndarray) -> np.ndarray:
        out = np.ascontiguousarray(hc, np.float32).copy()
        self.lib.orc_hc_add(_p(out, _f32p), _p(np.ascontiguousarray(block, np.float32), _f32p), block.size)
        return out


class RefLib:
    """The reference's own CPU path (oracle/_ref/libaffref.so)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (make -C oracle ref, needs the reference tree)")
        L = self.lib = C.CDLL(path)
        L.affref_collect_samples.argtypes = [_f32p, C.c_uint64, C.c_uint64, C.c_uint64, _f32p, C.c_uint64]
        L.affref_collect_samples.restype = C.c_uint64
        L.affref_fit_codebook.argtypes = [_f32p, C.c_uint64, C.c_uint32, C.c_uint64, C.c_int, _f32p]
        L.affref_pack_codebook.argtypes = [_f32p, _u32p]
        L.affref_unpack_codebook.argtypes = [_u32p, _f32p]
        L.affref_search_new.argtypes = [_f32p]
        L.affref_search_new.restype = C.c_void_p
        L.affref_search_free.argtypes = [C.c_void_p]
        L.affref_quantize_matrix.argtypes = [_f32p, C.c_uint64, C.c_uint64, _f32p, _f32p, C.c_void_p,
                                             _u8p, _u8p, _u8p]
        L.affref_quantize_matrix.restype = C.c_int
        L.affref_dequantize_matrix.argtypes = [_u8p, _u8p, _u8p, C.c_uint64, C.c_uint64, _f32p, _f32p]
        L.affref_dequantize_matrix.restype = C.c_int
        L.affref_expert_gemv_scaled.argtypes = [_u8p, _u8p, _u8p, C.c_uint64, C.c_uint64, _f32p, _f32p,
                                                C.c_float, _f32p, C.c_int]
        L.affref_swiglu.argtypes = [_f32p, _f32p, C.c_uint64, C.c_float, _f32p]
        L.affref_e4m3_to_float.argtypes = [C.c_uint8]
        L.affref_e4m3_to_float.restype = C.c_float
        L.affref_float_to_bf16.argtypes = [C.c_float]
        L.affref_float_to_bf16.restype = C.c_uint16
        L.affref_expert_layout.argtypes = [C.c_uint64, C.c_uint64, _u64p, _u64p]
        L.affref_expert_layout.restype = C.c_uint64
        L.affref_route_topk.argtypes = [_f32p, _f32p, C.c_uint32, C.c_uint32, C.c_int, C.c_float, _u32p, _f32p]
        L.affref_route_topk.restype = C.c_uint32
        L.affref_pool_threads.restype = C.c_uint
        L.affref_write_container.argtypes = [C.c_char_p, C.c_char_p, C.c_uint32, C.c_uint32, C.c_uint64, C.c_uint64,
                                             _u32p, _u8p, C.c_uint64, C.c_char_p, C.c_uint64]
        L.affref_write_container.restype = C.c_int
        L.affref_expert_offset.argtypes = [C.c_char_p, C.c_uint32, C.c_uint32]
        L.affref_expert_offset.restype = C.c_int64
        L.affref_matvec_fp8.argtypes = [_u8p, _u8p, C.c_uint64, C.c_uint64, _f32p, _f32p]
        L.affref_e8m0_to_float.argtypes = [C.c_uint8]
        L.affref_e8m0_to_float.restype = C.c_float
        L.affref_hc_expand.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_uint32, C.c_uint32]

    def collect_samples(self, w: np.ndarray, budget: int) -> np.ndarray:
        rows, cols = w.shape
        n = self.lib.affref_collect_samples(_p(w, _f32p), rows, cols, budget, None, 0)
        out = np.empty(n, np.float32)
        self.lib.affref_collect_samples(_p(w, _f32p), rows, cols, budget, _p(out, _f32p), n)
        return out

    def fit_codebook(self, samples, iters=50, seed=1, project=True) -> np.ndarray:
        cb = np.zeros(N_CB, np.float32)
        self.lib.affref_fit_codebook(_p(samples, _f32p), samples.size, iters, seed, int(project),
                                     _p(cb, _f32p))
        return cb

    def pack_codebook(self, cb) -> np.ndarray:
        out = np.zeros(2048, np.uint32)
        self.lib.affref_pack_codebook(_p(np.ascontiguousarray(cb, np.float32), _f32p), _p(out, _u32p))
        return out

    def unpack_codebook(self, packed) -> np.ndarray:
        out = np.zeros(N_CB, np.float32)
        self.lib.affref_unpack_codebook(_p(np.ascontiguousarray(packed, np.uint32), _u32p), _p(out, _f32p))
        return out

    def quantize(self, w: np.ndarray, cb: np.ndarray, importance=None, search: bool = True):
        rows, cols = w.shape
        nc, nf, _ = plane_bytes(rows, cols)
        codes = np.zeros(nc, np.uint8)
        fields = np.zeros(nf, np.uint8)
        rs = np.zeros(rows, np.uint16)
        h = self.lib.affref_search_new(_p(cb, _f32p)) if search else None
        try:
            imp = None if importance is None else _p(np.ascontiguousarray(importance, np.float32), _f32p)
            rc = self.lib.affref_quantize_matrix(_p(np.ascontiguousarray(w, np.float32), _f32p), rows,
                                                 cols, _p(cb, _f32p), imp, h, _p(codes, _u8p),
                                                 _p(fields, _u8p), rs.ctypes.data_as(_u8p))
        finally:
            if h:
                self.lib.affref_search_free(h)
        if rc != 0:
            raise ValueError("reference quantize_matrix refused the input")
        return codes, fields, rs

    def dequantize(self, codes, fields, rs, rows, cols, cb) -> np.ndarray:
        out = np.empty((rows, cols), np.float32)
        rc = self.lib.affref_dequantize_matrix(_p(codes, _u8p), _p(fields, _u8p), rs.ctypes.data_as(_u8p),
                                               rows, cols, _p(cb, _f32p), _p(out, _f32p))
        if rc != 0:
            raise ValueError("reference dequantize_matrix refused the input")
        return out

    def gemv(self, codes, fields, rs, rows, cols, cb, x, w=1.0, y=None, mt=False) -> np.ndarray:
        y = np.zeros(rows, np.float32) if y is None else y
        self.lib.affref_expert_gemv_scaled(_p(codes, _u8p), _p(fields, _u8p), rs.ctypes.data_as(_u8p),
                                           rows, cols, _p(cb, _f32p),
                                           _p(np.ascontiguousarray(x, np.float32), _f32p), float(w),
                                           _p(y, _f32p), int(mt))
        return y

    def route_topk(self, logits, bias, k=6, norm=True, scaling=1.0):
        sel = np.zeros(k, np.uint32)
        w = np.zeros(k, np.float32)
        lg = np.ascontiguousarray(logits, np.float32)
        b = None if bias is None else _p(np.ascontiguousarray(bias, np.float32), _f32p)
        n = self.lib.affref_route_topk(_p(lg, _f32p), b, lg.size, k, int(norm), scaling, _p(sel, _u32p),
                                       _p(w, _f32p))
        return sel[:n], w[:n]

    def write_container(self, path: str, meta: str, experts: np.ndarray, codebook: np.ndarray, hidden: int,
                        inter: int) -> None:
        """A .aff file through the reference's AffWriter. experts: uint8 [layers][experts][stride]."""
        n_layers, n_experts, stride = experts.shape
        err = C.create_string_buffer(512)
        rc = self.lib.affref_write_container(path.encode(), meta.encode(), n_layers, n_experts, hidden, inter,
                                             _p(np.ascontiguousarray(codebook, np.uint32), _u32p),
                                             _p(np.ascontiguousarray(experts), _u8p), stride, err, 512)
        if rc != 0:
            raise ValueError("reference AffWriter: " + err.value.decode())

    def expert_offset(self, path: str, layer: int, expert: int) -> int:
        """File offset of an expert by the reference reader's own addressing."""
        return int(self.lib.affref_expert_offset(path.encode(), layer, expert))

    def pool_threads(self) -> int:
        """Threads of the reference's global pool (hardware_concurrency), which the _mt GEMV uses."""
        return int(self.lib.affref_pool_threads())

    def swiglu(self, g, u, limit=10.0) -> np.ndarray:
        out = np.empty_like(g, dtype=np.float32)
        self.lib.affref_swiglu(_p(g, _f32p), _p(u, _f32p), g.size, limit, _p(out, _f32p))
        return out

    def e4m3_to_float(self, b: int) -> float:
        return float(self.lib.affref_e4m3_to_float(b))

    def e8m0_to_float(self, b: int) -> float:
        return float(self.lib.affref_e8m0_to_float(b))

    def matvec_fp8(self, w: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
        rows, cols = w.shape
        out = np.zeros(rows, np.float32)
        self.lib.affref_matvec_fp8(_p(w, _u8p), _p(s, _u8p), rows, cols,
                                   _p(np.ascontiguousarray(x, np.float32), _f32p), _p(out, _f32p))
        return out

    def hc_expand(self, block, hc, post, comb) -> np.ndarray:
        n_hc, n = hc.shape
        out = np.zeros((n_hc, n), np.float32)
        self.lib.affref_hc_expand(_p(out, _f32p), _p(np.ascontiguousarray(block, np.float32), _f32p),
                                  _p(np.ascontiguousarray(hc, np.float32), _f32p),
                                  _p(np.ascontiguousarray(post, np.float32), _f32p),
                                  _p(np.ascontiguousarray(comb, np.float32), _f32p), n, n_hc)
        return out

    def float_to_bf16(self, f: float) -> int:
        return int(self.lib.affref_float_to_bf16(f))

    def expert_layout(self, hidden: int = H, inter: int = I):
        off = np.zeros(9, np.uint64)
        size = np.zeros(9, np.uint64)
        stride = self.lib.affref_expert_layout(hidden, inter, _p(off, _u64p), _p(size, _u64p))
        return int(stride), off.astype(np.int64), size.astype(np.int64)


_oracle = None
_ref = None


def load_oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def load_ref() -> RefLib:
    global _ref
    if _ref is None:
        _ref = RefLib()
    return _ref
