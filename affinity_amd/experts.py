"""Host-side mirror of the reference's routed-expert interface, over libaffx.so.

The reference keeps its experts in one device slab, addressed expert e of a layer at
base + e*stride (src/format/aff_reader.h:45-48; StaticPlacement, src/gpu/static_placement.hip:
745-1100), and runs them through the entry points of src/gpu/expert_kernel_hip.h. Here an
`ExpertPool` is that slab for one layer in the device layout, and the functions below are the
entry points, taking torch tensors for device memory and streams (plumbing only: the compute is
the HIP library). There is no CPU fallback: every function raises when the library is missing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import AffxLayer, AffxMatrix, check, lib

HIDDEN, INTER, N_EXPERTS, TOP_K, SWIGLU_LIMIT = 4096, 2048, 256, 6, 10.0   # src/engine/model.h:23-53


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def init() -> None:
    check(lib().affx_init(), "affx_init")


def expert_layout(hidden: int = HIDDEN, inter: int = INTER):
    """(stride, plane offsets[9], plane sizes[9]); planes ordered gate/up/down x codes/fields/rscales."""
    off = (C.c_uint64 * 9)()
    size = (C.c_uint64 * 9)()
    stride = lib().affx_expert_layout(hidden, inter, off, size)
    return int(stride), list(off), list(size)


def e4m3_table() -> np.ndarray:
    """OCP E4M3 'fn' decode table (bias 7, no infinities, S.1111.111 = NaN)."""
    b = np.arange(256)
    e, m = (b >> 3) & 15, b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(b & 0x80, -v, v).astype(np.float32)


def codebook_floats(packed: np.ndarray) -> np.ndarray:
    """uint32[2048] packed E4M3 quads -> float32[2][1024][4] (the quantiser's search table)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    t = e4m3_table()
    by = packed.view(np.uint8).reshape(2048, 4)
    return t[by].reshape(2, 1024, 4).astype(np.float32)


def codebook_valid(packed: np.ndarray) -> bool:
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    return bool(lib().affx_codebook_valid(packed.ctypes.data))


@dataclass
class ExpertPool:
    """One layer's routed experts, resident in HBM in device layout."""

    data: torch.Tensor           # uint8 [n_experts * stride]
    codebook: torch.Tensor       # int32 [2048] (packed E4M3 quads)
    n_experts: int
    hidden: int = HIDDEN
    inter: int = INTER
    swiglu_limit: float = SWIGLU_LIMIT

    @property
    def stride(self) -> int:
        return expert_layout(self.hidden, self.inter)[0]

    @classmethod
    def empty(cls, n_experts: int, codebook_packed: np.ndarray, hidden: int = HIDDEN,
              inter: int = INTER, device: str = "cuda", swiglu_limit: float = SWIGLU_LIMIT):
        if not codebook_valid(codebook_packed):
            raise _lib.AffxError("codebook has a stored exponent outside 1..7")
        stride = expert_layout(hidden, inter)[0]
        data = torch.empty(n_experts * stride, dtype=torch.uint8, device=device)
        cb = torch.from_numpy(np.ascontiguousarray(codebook_packed, np.uint32).view(np.int32)).to(device)
        return cls(data, cb, n_experts, hidden, inter, swiglu_limit)

    @classmethod
    def from_container(cls, container: torch.Tensor, codebook_packed: np.ndarray,
                       hidden: int = HIDDEN, inter: int = INTER, stream=None,
                       swiglu_limit: float = SWIGLU_LIMIT):
        """Upload experts given in the container layout (a uint8 tensor of n*stride bytes, host or
        device) and permute them into the device layout on the GPU."""
        stride = expert_layout(hidden, inter)[0]
        assert container.numel() % stride == 0, "container bytes must be whole experts"
        n = container.numel() // stride
        pool = cls.empty(n, codebook_packed, hidden, inter, swiglu_limit=swiglu_limit)
        src = container.to(pool.data.device, non_blocking=False).contiguous()
        check(lib().affx_permute_experts(src.data_ptr(), pool.data.data_ptr(), n, hidden, inter,
                                         _stream(stream)), "affx_permute_experts")
        torch.cuda.current_stream().synchronize() if stream is None else None
        return pool

    def layer(self) -> AffxLayer:
        return AffxLayer(self.data.data_ptr(), self.stride, self.n_experts, self.hidden, self.inter,
                         self.codebook.data_ptr(), self.swiglu_limit)

    def matrix(self, expert: int, which: int) -> AffxMatrix:
        """which: 0 gate, 1 up, 2 down."""
        stride, off, _ = expert_layout(self.hidden, self.inter)
        base = self.data.data_ptr() + expert * stride
        rows = (self.inter, self.inter, self.hidden)[which]
        cols = (self.hidden, self.hidden, self.inter)[which]
        return AffxMatrix(base + off[3 * which], base + off[3 * which + 1], base + off[3 * which + 2],
                          rows, cols)


def dequant_matrix(pool: ExpertPool, expert: int, which: int, stream=None) -> torch.Tensor:
    m = pool.matrix(expert, which)
    out = torch.empty((m.rows, m.cols), dtype=torch.float32, device=pool.data.device)
    check(lib().affx_dequant_matrix(C.byref(m), pool.codebook.data_ptr(), out.data_ptr(),
                                    _stream(stream)), "affx_dequant_matrix")
    return out


class DecodeWorkspace:
    def __init__(self, m_tokens: int, top_k: int, hidden: int = HIDDEN, inter: int = INTER,
                 device="cuda"):
        self.bytes = int(lib().affx_decode_workspace_size(m_tokens, top_k, hidden, inter))
        # zero-filled: the fused decode keeps its cross-workgroup counter and release flags at the
        # start of the workspace and expects them zero on first use (each launch leaves them zero)
        self.buf = torch.zeros(self.bytes, dtype=torch.uint8, device=device)

    def error_flags(self) -> int:
        """Nonzero if a fused decode launch on this workspace gave up waiting (bounded spin)."""
        return int(self.buf[8:12].view(torch.int32).item())

    def status(self, reset: bool = False, stream=None) -> int:
        """affx_decode_status: 0, or AFFX_ERR_DEVICE (< 0) when a launch on this workspace gave up
        waiting for its workgroups; reset zeroes the sync run. Synchronises the stream."""
        return int(lib().affx_decode_status(self.buf.data_ptr(), int(reset), _stream(stream)))


def expert_ffn_decode(pool: ExpertPool, x: torch.Tensor, sel: torch.Tensor, w: torch.Tensor,
                      y: torch.Tensor | None = None, accumulate: bool = False,
                      workspace: DecodeWorkspace | None = None, stream=None,
                      dim_major: bool = False, staged: bool = False) -> torch.Tensor:
    """y[t] (+)= sum_j w[t,j] * FFN_{sel[t,j]}(x[t]) for M <= 8 tokens.

    x: f32 [M, hidden] (token-major) or, with dim_major, [hidden, M] (the engine's d_x arena).
    sel: int32/uint32 [M, k] device; w: f32 [M, k] device.
    staged: the three-launch form (affx_decode_staged) instead of the one persistent launch.
    """
    if dim_major:
        hidden, M = x.shape
        xts, xds = 1, x.stride(0)
    else:
        M, hidden = x.shape
        xts, xds = x.stride(0), 1
    k = sel.shape[1]
    if y is None:
        y = torch.zeros_like(x)
    yts, yds = (1, y.stride(0)) if dim_major else (y.stride(0), 1)
    ws = workspace or DecodeWorkspace(M, k, pool.hidden, pool.inter, device=x.device)
    L = pool.layer()
    sel = sel.contiguous()
    w = w.contiguous()
    fn = lib().affx_decode_staged if staged else lib().affx_expert_ffn_decode
    check(fn(C.byref(L), x.data_ptr(), xts, xds, M, sel.data_ptr(), w.data_ptr(), k, y.data_ptr(), yts,
             yds, int(accumulate), ws.buf.data_ptr(), ws.bytes, _stream(stream)),
          "affx_decode_staged" if staged else "affx_expert_ffn_decode")
    return y


class GroupedWorkspace:
    def __init__(self, n_tok: int, top_k: int, n_experts: int, hidden: int = HIDDEN,
                 inter: int = INTER, device="cuda"):
        self.bytes = int(lib().affx_grouped_workspace_size(n_tok, top_k, n_experts, hidden, inter))
        self.buf = torch.empty(self.bytes, dtype=torch.uint8, device=device)


def expert_ffn_grouped(pool: ExpertPool, x: torch.Tensor, sel: torch.Tensor, w: torch.Tensor,
                       y: torch.Tensor | None = None, accumulate: bool = False,
                       x_lo: torch.Tensor | None = None, workspace: GroupedWorkspace | None = None,
                       stream=None) -> torch.Tensor:
    """Prefill: y[t] (+)= sum_j w[t,j] * FFN_{sel[t,j]}(x[t]) for all tokens, grouped by expert.

    x: bf16 [T, hidden] token-major (x_lo: optional second bf16 term); y: f32 [T, hidden].
    """
    T, hidden = x.shape
    k = sel.shape[1]
    if y is None:
        y = torch.zeros((T, hidden), dtype=torch.float32, device=x.device)
    ws = workspace or GroupedWorkspace(T, k, pool.n_experts, pool.hidden, pool.inter, device=x.device)
    L = pool.layer()
    x = x.contiguous()
    check(lib().affx_expert_ffn_grouped(C.byref(L), x.data_ptr(),
                                        0 if x_lo is None else x_lo.contiguous().data_ptr(), T,
                                        sel.contiguous().data_ptr(), w.contiguous().data_ptr(), k,
                                        y.data_ptr(), int(accumulate), ws.buf.data_ptr(), ws.bytes,
                                        _stream(stream)), "affx_expert_ffn_grouped")
    return y


def quantize_matrix(w: torch.Tensor, codebook_f32: torch.Tensor, importance: torch.Tensor | None = None,
                    stream=None):
    """GPU quantiser: f32 [rows, cols] -> (codes, fields, rscales) in the container's row-major
    bit streams, bit-identical to the reference's quantize_matrix."""
    rows, cols = w.shape
    codes = torch.empty(rows * cols * 10 // 32, dtype=torch.uint8, device=w.device)
    fields = torch.empty(rows * cols * 6 // 128, dtype=torch.uint8, device=w.device)
    rs = torch.empty(rows, dtype=torch.int16, device=w.device)
    check(lib().affx_quantize_matrix(w.contiguous().data_ptr(), rows, cols, codebook_f32.data_ptr(),
                                     0 if importance is None else importance.data_ptr(),
                                     codes.data_ptr(), fields.data_ptr(), rs.data_ptr(),
                                     _stream(stream)), "affx_quantize_matrix")
    return codes, fields, rs


def gen_normal(seed: int, n: int, scale: float = 1.0, bf16_round: bool = True, device="cuda",
               stream=None) -> torch.Tensor:
    out = torch.empty(n, dtype=torch.float32, device=device)
    check(lib().affx_gen_normal(seed, n, scale, out.data_ptr(), int(bf16_round), _stream(stream)),
          "affx_gen_normal")
    return out


def fill_synthetic_experts(container: torch.Tensor, first: int, count: int, codebook_f32: torch.Tensor,
                           seed_of, hidden: int = HIDDEN, inter: int = INTER, stream=None) -> None:
    """Writes `count` synthetic experts (container layout) starting at expert `first` of the
    uint8 device buffer `container`; expert e gets seeds seed_of(e) + {0,1,2}."""
    stride = expert_layout(hidden, inter)[0]
    scratch = torch.empty(hidden * inter, dtype=torch.float32, device=container.device)
    for e in range(first, first + count):
        check(lib().affx_fill_expert(container.data_ptr() + e * stride, hidden, inter,
                                     codebook_f32.data_ptr(), int(seed_of(e)), scratch.data_ptr(),
                                     _stream(stream)), "affx_fill_expert")


# ---- the step after: shared expert and hyper-connection post ------------------------------------

def dense_fp8_to_device_layout(w: torch.Tensor, stream=None) -> torch.Tensor:
    """The container's row-major E4M3 bytes [rows x cols] (uint8, on the device) in the device
    layout the shared-expert kernels read (a new tensor of the same shape)."""
    out = torch.empty_like(w)
    check(lib().affx_dense_fp8_to_device_layout(w.contiguous().data_ptr(), out.data_ptr(), w.shape[0], w.shape[1],
                                                _stream(stream)), "dense_fp8_to_device_layout")
    return out


class SharedExpert:
    """A layer's FP8 shared expert on the device (the reference's shexp_gate/up/down DenseW,
    src/engine/model.h:125-127): E4M3 weights [rows x cols] (uint8 tensors, row-major as the
    container holds them; permuted here into the device layout) and UE8M0 tile scales
    [rows / 128][cols / 128]."""

    def __init__(self, gate, gate_s, up, up_s, down, down_s, swiglu_limit: float = SWIGLU_LIMIT):
        inter, hidden = gate.shape
        gate, up, down = (dense_fp8_to_device_layout(m) for m in (gate, up, down))
        self.tensors = (gate, gate_s, up, up_s, down, down_s)   # keeps the memory alive
        mk = lambda w, s: _lib.AffxDenseFp8(w.data_ptr(), s.data_ptr(), w.shape[0], w.shape[1])
        self.abi = _lib.AffxSharedExpert(mk(gate, gate_s), mk(up, up_s), mk(down, down_s), hidden, inter,
                                         float(swiglu_limit))
        self.hidden, self.inter = hidden, inter

    def decode(self, x: torch.Tensor, y: torch.Tensor, accumulate: bool = True, stream=None) -> torch.Tensor:
        """y (+)= W_d . swiglu(W_g x, W_u x) for M <= 8 f32 tokens x [M][hidden] (DenseOps::shexp,
        src/engine/model.h:314-319)."""
        M = x.shape[0]
        ws = torch.empty(lib().affx_shared_decode_workspace_size(M, self.hidden, self.inter), dtype=torch.uint8,
                         device=x.device)
        check(lib().affx_shared_expert_decode(C.byref(self.abi), x.data_ptr(), x.stride(0), x.stride(1), M,
                                              y.data_ptr(), y.stride(0), y.stride(1), int(accumulate),
                                              ws.data_ptr(), ws.numel(), _stream(stream)), "shared_expert_decode")
        return y

    def batch(self, x: torch.Tensor, y: torch.Tensor, x_lo: torch.Tensor | None = None, accumulate: bool = True,
              stream=None) -> torch.Tensor:
        """y (+)= the shared expert of every bf16 token row of x [T][hidden] (BatchOps::shexp,
        src/engine/model.h:504-505)."""
        T = x.shape[0]
        ws = torch.empty(lib().affx_shared_batch_workspace_size(T, self.hidden, self.inter), dtype=torch.uint8,
                         device=x.device)
        check(lib().affx_shared_expert_batch(C.byref(self.abi), x.data_ptr(), 0 if x_lo is None else x_lo.data_ptr(),
                                             T, y.data_ptr(), int(accumulate), ws.data_ptr(), ws.numel(),
                                             _stream(stream)), "shared_expert_batch")
        return y


def hc_post(block: torch.Tensor, hc: torch.Tensor, post: torch.Tensor | None, comb: torch.Tensor | None,
            out_hc: torch.Tensor | None = None, zero_block: bool = True, stream=None) -> torch.Tensor:
    """The sublayer's hyper-connection post for one token (DenseGpu::hc_post,
    src/gpu/dense_gpu.hip:2394-2465): with a control (post, comb) the next state
    [n_hc][n_embd] = block * post[dst] + sum_src comb[dst + src n_hc] * hc[src]; without one,
    hc[0] += block in place. The block is left zero when zero_block."""
    n_hc, n = hc.shape
    s = _stream(stream)
    if post is None:
        check(lib().affx_hc_add(hc.data_ptr(), block.data_ptr(), n, int(zero_block), s), "hc_add")
        return hc
    out_hc = torch.empty_like(hc) if out_hc is None else out_hc
    check(lib().affx_hc_post(out_hc.data_ptr(), block.data_ptr(), hc.data_ptr(), post.data_ptr(), comb.data_ptr(),
                             n, n_hc, int(zero_block), s), "hc_post")
    return out_hc


def hc_post_batch(block: torch.Tensor, hc: torch.Tensor, post: torch.Tensor | None, comb: torch.Tensor | None,
                  out_hc: torch.Tensor | None = None, zero_block: bool = True, stream=None) -> torch.Tensor:
    """The batch form over the engine's dim-major arenas (batch_hc_post, src/gpu/dense_gpu.hip:
    4517-4534): hc bf16 [n_hc][n_embd][nb], block f32 [n_embd][nb], post [n_hc][nb], comb
    [n_hc * n_hc][nb]; without a control hc lane 0 += block in place."""
    n_hc, n, nb = hc.shape
    s = _stream(stream)
    if post is None:
        check(lib().affx_hc_add_batch(hc.data_ptr(), block.data_ptr(), n * nb, int(zero_block), s), "hc_add_batch")
        return hc
    out_hc = torch.empty_like(hc) if out_hc is None else out_hc
    check(lib().affx_hc_post_batch(out_hc.data_ptr(), block.data_ptr(), hc.data_ptr(), post.data_ptr(),
                                   comb.data_ptr(), n, n_hc, nb, int(zero_block), s), "hc_post_batch")
    return out_hc
