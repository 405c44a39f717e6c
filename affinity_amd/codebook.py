"""The codebook producer on the GPU, over libaffx.so: the functions aff-quantize runs before it
quantises (src/quant/blockquant.h:131-175; called at tools/aff_quantize.cpp:391, 420-434, 519),
for the quad format (4-wide codes, 1024 entries, 2 variants, power-of-two block scales).

Tensors are device memory (torch is plumbing only); every result equals the reference CPU path's
bit for bit. There is no CPU fallback: every function raises when the library is missing.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import check, lib
from .experts import _stream

N_VARIANTS, N_ENTRIES = 2, 1024
SEQUENTIAL_PICKS = 1   # AFFX_FIT_SEQUENTIAL_PICKS


def collect_normalized_samples(w: torch.Tensor, max_samples: int = 1 << 22, stream=None) -> torch.Tensor:
    """collect_normalized_samples (blockquant.cpp:386-423) of a row-major f32 matrix on the device,
    without importance: every stride-th row, each nonzero 16-block divided by its max |w|."""
    if w.dtype != torch.float32 or w.dim() != 2 or not w.is_cuda:
        raise ValueError("collect_normalized_samples: w must be a 2-D float32 CUDA tensor")
    w = w.contiguous()
    rows, cols = w.shape
    L = lib()
    bound = int(L.affx_collect_samples_bound(rows, cols, max_samples))
    out = torch.empty(max(bound, 4), dtype=torch.float32, device=w.device)
    n_out = torch.zeros(1, dtype=torch.int64, device=w.device)
    ws = torch.empty(int(L.affx_collect_samples_workspace_size(rows, cols, max_samples)), dtype=torch.uint8,
                     device=w.device)
    check(L.affx_collect_samples(w.data_ptr(), rows, cols, max_samples, out.data_ptr(), out.numel(),
                                 n_out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(stream)),
          "collect_normalized_samples")
    n = int(n_out.item())
    if n > out.numel():
        raise RuntimeError(f"collect_normalized_samples: {n} samples exceed the bound {out.numel()}")
    return out[:n]


class CodebookFit:
    """fit_codebook (blockquant.cpp:252-384) with the workspace kept for repeated fits and for
    the counters of the last one."""

    def __init__(self, n_samples: int, device="cuda"):
        self.n_samples = int(n_samples)
        self.ws = torch.empty(int(lib().affx_fit_codebook_workspace_size(self.n_samples)) + 256, dtype=torch.uint8,
                              device=device)
        off = (-self.ws.data_ptr()) % 256
        self.ws_ptr, self.ws_bytes = self.ws.data_ptr() + off, self.ws.numel() - off

    def fit(self, samples: torch.Tensor, iters: int = 50, seed: int = 1, flags: int = 0,
            stream=None) -> torch.Tensor:
        """The raw joint fit, float32 [2][1024][4] on the device (before projection)."""
        if samples.dtype != torch.float32 or not samples.is_cuda:
            raise ValueError("fit_codebook: samples must be a float32 CUDA tensor")
        samples = samples.contiguous()
        if samples.numel() > self.n_samples:
            raise ValueError("fit_codebook: more samples than the workspace was sized for")
        if samples.data_ptr() % 16:
            samples = samples.clone()
        cb = torch.empty((N_VARIANTS, N_ENTRIES, 4), dtype=torch.float32, device=samples.device)
        check(lib().affx_fit_codebook(samples.data_ptr(), samples.numel(), None, iters, seed, flags, cb.data_ptr(),
                                      self.ws_ptr, self.ws_bytes, _stream(stream)), "fit_codebook")
        return cb

    def stats(self, stream=None) -> tuple[int, int]:
        """(k-means++ draws taken by the sequential sums, Lloyd passes) of the last fit."""
        a, b = C.c_uint64(), C.c_uint64()
        check(lib().affx_fit_codebook_stats(self.ws_ptr, C.byref(a), C.byref(b), _stream(stream)),
              "fit_codebook_stats")
        return int(a.value), int(b.value)


def fit_codebook(samples: torch.Tensor, iters: int = 50, seed: int = 1, flags: int = 0, stream=None) -> torch.Tensor:
    return CodebookFit(samples.numel(), samples.device).fit(samples, iters, seed, flags, stream)


def project_codebook_e4m3(cb: torch.Tensor, stream=None) -> torch.Tensor:
    """project_codebook_e4m3 (blockquant.cpp:463-466), pow2 scales, in place; returns cb."""
    if cb.dtype != torch.float32 or not cb.is_cuda or not cb.is_contiguous():
        raise ValueError("project_codebook_e4m3: cb must be a contiguous float32 CUDA tensor")
    check(lib().affx_project_codebook(cb.data_ptr(), cb.numel(), _stream(stream)), "project_codebook_e4m3")
    return cb


def pack_codebook_e4m3_quads(cb: torch.Tensor, stream=None) -> torch.Tensor:
    """pack_codebook_e4m3_quads (blockquant.cpp:468-480): int32 [2048] (the uint32 dwords)."""
    if cb.dtype != torch.float32 or not cb.is_cuda or cb.numel() != N_VARIANTS * N_ENTRIES * 4:
        raise ValueError("pack_codebook_e4m3_quads: cb must be float32 [2][1024][4] on the device")
    cb = cb.contiguous()
    out = torch.empty(N_VARIANTS * N_ENTRIES, dtype=torch.int32, device=cb.device)
    check(lib().affx_pack_codebook(cb.data_ptr(), out.data_ptr(), _stream(stream)), "pack_codebook_e4m3_quads")
    return out


def unpack_codebook_e4m3_quads(packed: torch.Tensor, stream=None) -> torch.Tensor:
    """unpack_codebook_e4m3_quads (blockquant.cpp:482-492): float32 [2][1024][4]."""
    if packed.dtype != torch.int32 or not packed.is_cuda or packed.numel() != N_VARIANTS * N_ENTRIES:
        raise ValueError("unpack_codebook_e4m3_quads: packed must be int32 [2048] on the device")
    packed = packed.contiguous()
    cb = torch.empty((N_VARIANTS, N_ENTRIES, 4), dtype=torch.float32, device=packed.device)
    check(lib().affx_unpack_codebook(packed.data_ptr(), cb.data_ptr(), _stream(stream)), "unpack_codebook_e4m3_quads")
    return cb
