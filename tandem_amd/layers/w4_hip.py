"""Load libtandem_w4.so (the gfx950 W4A16 kernels, C ABI in include/tandem_w4.h) and own the split-K
workspace: the MI355X counterpart of python/tandem/layers/w4_cuda.py.

The reference JIT-builds a torch extension with nvcc on first use (w4_cuda.py:44-62) and falls back
to dequantize + cuBLAS when that fails. Here the library is built ahead of time, in-tree
(``python -m tandem_amd.build``), and there is no silent fallback: if it is missing, every call
raises. ``load()`` returns None only when ``TANDEM_NO_CUDA_EXT=1`` switches the fused kernels off
(w4_cuda.py:46), which sends W4Linear to the HIP dequantize kernel + torch.matmul.

``load()`` returns an object with the reference extension's three entry points and argument order
(w4_cuda.py:17-21): ``w4_gemv(x, w, s, z, warps_k, unroll, ntile)``, ``w4_mma(x, w, s, z, warps_k,
unroll, ntile, act)``, ``w4_gemm(x, w, s, z, ws, locks, mt, nt, warps_n, warps_k, stages, splits,
act)``; each allocates y with torch on x's device and launches on the current stream.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libtandem_w4.so")

TW4_OK, TW4_EINVAL, TW4_ECONFIG, TW4_EHIP, TW4_ESPACE = 0, 1, 2, 3, 4

WORKSPACE_FLOATS = 1 << 23  # 32 MB of float32 split-K partial sums per GPU (w4_cuda.py:24)
WORKSPACE_LOCKS = 1 << 15
_workspaces: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
_init_lock = threading.Lock()
_initialized: set[int] = set()

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SIGNATURES = {
    "tw4_version": ([], ctypes.c_char_p),
    "tw4_arch": ([], ctypes.c_char_p),
    "tw4_last_error": ([], ctypes.c_char_p),
    "tw4_init": ([_I], _I),
    "tw4_repack_awq": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _P], _I),
    "tw4_dequant": ([_P, _P, _P, _P, _I, _I, _I, _P], _I),
    "tw4_gemv": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemv_act": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemv_mfma": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_mma": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_mma_splitk": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_mma_persist": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemm": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemm_noalloc": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemm_last_grid": ([ctypes.POINTER(_I)] * 3, _I),
    "tw4_read_probe": ([_P, _I64, _I, _I, _I, ctypes.c_uint32, _P, _P], _I),
    "tw4_decode_configs": ([ctypes.POINTER(_I), _I], _I),
    "tw4_mma_wide_configs": ([ctypes.POINTER(_I), _I], _I),
    "tw4_gemm_configs": ([ctypes.POINTER(_I), _I], _I),
    "tw4_gemv_f16": ([_P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "tw4_gemv_f16_configs": ([ctypes.POINTER(_I), _I], _I),
    "tw4_decode_norm": ([_P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "tw4_rms_norm": ([_P, _P, _P, _I, _I, ctypes.c_float, _P], _I),
    "tw4_add_rms_norm": ([_P, _P, _P, _I, _I, ctypes.c_float, _P], _I),
}


@functools.lru_cache(maxsize=None)
def library() -> ctypes.CDLL:
    """The C-ABI library with argument types set. Raises RuntimeError if it is not built."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m tandem_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _configs(name: str, width: int) -> tuple[tuple[int, ...], ...]:
    fn = getattr(library(), name)
    n = fn(None, 0)
    buf = (_I * (width * n))()
    fn(buf, n)
    return tuple(tuple(buf[width * i + j] for j in range(width)) for i in range(n))


def decode_configs() -> tuple[tuple[int, int, int], ...]:
    """The compiled (warps_k, unroll, ntile) configurations of w4_gemv / w4_mma."""
    return _configs("tw4_decode_configs", 3)


def mma_wide_configs() -> tuple[tuple[int, int, int], ...]:
    """The row-tile-wide (warps_k, unroll, ntile) configurations only w4_mma takes (x read from global
    memory, up to six row tiles per workgroup; no split-K, persistent form or fused norm)."""
    return _configs("tw4_mma_wide_configs", 3)


def mma_configs() -> tuple[tuple[int, int, int], ...]:
    """Every (warps_k, unroll, ntile) configuration w4_mma takes."""
    return decode_configs() + mma_wide_configs()


def gemm_configs() -> tuple[tuple[int, int, int, int, int], ...]:
    """The compiled (mt, nt, warps_n, warps_k, stages) configurations of w4_gemm."""
    return _configs("tw4_gemm_configs", 5)


def gemv_f16_configs() -> tuple[tuple[int, int], ...]:
    """The compiled (rows in flight, rows per wavefront) configurations of tw4_gemv_f16."""
    return _configs("tw4_gemv_f16_configs", 2)


def check(status: int) -> None:
    """Map a TW4_* status to the reference's exception type (TORCH_CHECK -> RuntimeError)."""
    if status != TW4_OK:
        msg = library().tw4_last_error().decode(errors="replace")
        raise RuntimeError(f"tandem_w4: {msg} (status {status})")


def init_device(device: torch.device | int) -> None:
    """tw4_init once per device, before any graph capture (kernel attributes, occupancy)."""
    index = device if isinstance(device, int) else (device.index if device.index is not None
                                                     else torch.cuda.current_device())
    if index in _initialized:
        return
    with _init_lock:
        if index not in _initialized:
            check(library().tw4_init(index))
            _initialized.add(index)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def padded_rows(n: int) -> int:
    return (n + 15) // 16 * 16


def check_operands(who: str, x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor) -> tuple[int, int, int]:
    """The reference extension's argument checks (python/tandem/csrc/w4_gemv.cu:568-579), for the
    tile layout: x [M, K] fp16 contiguous 16-byte aligned on a GPU; packed int32 [Npad, K/8];
    scales / zeros fp16 [N, K/128]. Returns (M, N, K). Never lets a CPU pointer reach a kernel."""
    if not (x.is_cuda and x.dim() == 2 and x.dtype == torch.float16 and x.is_contiguous()):
        raise RuntimeError(f"{who}: x must be a contiguous 2-D float16 GPU tensor")
    if x.data_ptr() % 16:
        raise RuntimeError(f"{who}: x must be 16-byte aligned")
    if not (w.is_cuda and w.dtype == torch.int32 and w.is_contiguous() and w.data_ptr() % 16 == 0):
        raise RuntimeError(f"{who}: packed must be a contiguous 16-byte aligned int32 GPU tensor")
    if not (s.is_cuda and z.is_cuda and s.dtype == torch.float16 and z.dtype == torch.float16
            and s.is_contiguous() and z.is_contiguous()):
        raise RuntimeError(f"{who}: scales / zeros must be contiguous float16 GPU tensors")
    if not (x.device == w.device == s.device == z.device):
        raise RuntimeError(f"{who}: x, packed, scales and zeros must be on one device")
    m, k = x.shape
    if k % 128 or s.dim() != 2 or s.shape[1] * 128 != k or z.shape != s.shape:
        raise RuntimeError(f"{who}: K % 128 == 0 and scales / zeros [N, K / 128] (x {tuple(x.shape)}, "
                           f"scales {tuple(s.shape)}, zeros {tuple(z.shape)})")
    n = s.shape[0]
    if w.dim() != 2 or w.shape != (padded_rows(n), k // 8):
        raise RuntimeError(f"{who}: packed must be [{padded_rows(n)}, {k // 8}] (got {tuple(w.shape)})")
    return m, n, k


class W4Extension:
    """The reference extension's three kernels (python/tandem/csrc/w4_gemv.cu:604-683) over the C ABI."""

    def __init__(self) -> None:
        self.lib = library()

    def w4_gemv(self, x, w, s, z, warps_k: int, unroll: int, ntile: int, act: int = 0) -> torch.Tensor:
        """act = 1 (not in the reference's w4_gemv): the SwiGLU epilogue of w4_mma."""
        m, n, k = check_operands("w4_gemv", x, w, s, z)
        if not 1 <= m <= 4:
            raise RuntimeError("w4_gemv: M <= 4 (larger M: w4_mma)")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_gemv: act 0, or 1 (SwiGLU) with N % 16 == 0")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            check(self.lib.tw4_gemv_act(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), m, n, k,
                                        int(warps_k), int(unroll), int(ntile), int(act), _stream(x)))
        return y

    def w4_gemv_mfma(self, x, w, s, z, warps_k: int, unroll: int, ntile: int, act: int = 0) -> torch.Tensor:
        """The GEMV's arithmetic on the matrix cores (tw4_gemv_mfma; no reference counterpart), M <= 16
        (x' of M rows must fit in LDS: K = 4096 takes any M <= 16, K = 12288 M <= 4)."""
        m, n, k = check_operands("w4_gemv_mfma", x, w, s, z)
        if not 1 <= m <= 16:
            raise RuntimeError("w4_gemv_mfma: M <= 16 (larger M: w4_mma)")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_gemv_mfma: act 0, or 1 (SwiGLU) with N % 16 == 0")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            check(self.lib.tw4_gemv_mfma(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), m, n, k,
                                         int(warps_k), int(unroll), int(ntile), int(act), _stream(x)))
        return y

    def w4_decode_norm(self, x, residual, norm_weight, eps: float, w, s, z, kind: int, warps_k: int, unroll: int,
                       ntile: int, act: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        """w4_gemv (kind 0) / w4_mma (kind 1) of rms_norm(x + residual) * norm_weight, the norm fused
        into the kernel's x staging (tw4_decode_norm); returns (y, fp16(x + residual)), or (y, None)
        without a residual. Bit-identical to tw4_add_rms_norm / tw4_rms_norm, then the kernel."""
        m, n, k = check_operands("w4_decode_norm", x, w, s, z)
        if residual is not None and (residual.shape != x.shape or residual.dtype != torch.float16
                                     or not residual.is_contiguous() or residual.device != x.device):
            raise RuntimeError("w4_decode_norm: residual must be a contiguous float16 tensor like x")
        if (norm_weight.shape != (k,) or norm_weight.dtype != torch.float16 or norm_weight.device != x.device
                or not norm_weight.is_contiguous()):
            raise RuntimeError(f"w4_decode_norm: contiguous float16 norm weight [{k}] on x's GPU expected")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        r_out = torch.empty_like(x) if residual is not None else None
        with torch.cuda.device(x.device):
            check(self.lib.tw4_decode_norm(_ptr(x), _ptr(residual) if residual is not None else None,
                                           _ptr(r_out) if r_out is not None else None, _ptr(norm_weight), float(eps),
                                           _ptr(w), _ptr(s), _ptr(z), _ptr(y), m, n, k, int(kind), int(warps_k),
                                           int(unroll), int(ntile), int(act), _stream(x)))
        return y, r_out

    def w4_mma(self, x, w, s, z, warps_k: int, unroll: int, ntile: int, act: int) -> torch.Tensor:
        m, n, k = check_operands("w4_mma", x, w, s, z)
        if not 1 <= m <= 64:
            raise RuntimeError("w4_mma: M <= 64 (16-token batch tiles: 1, 2 or 4)")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_mma: act 0, or 1 (SwiGLU) with N % 16 == 0")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            check(self.lib.tw4_mma(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), m, n, k,
                                   int(warps_k), int(unroll), int(ntile), int(act), _stream(x)))
        return y

    def w4_mma_persist(self, x, w, s, z, warps_k: int, unroll: int, ntile: int, per_cu: int,
                       act: int) -> torch.Tensor:
        """w4_mma's persistent form (M <= 16, x in LDS): at most per_cu workgroups per CU, each staging
        x once and streaming several row-tile groups."""
        m, n, k = check_operands("w4_mma", x, w, s, z)
        if not 1 <= m <= 16:
            raise RuntimeError("w4_mma_persist: M <= 16 (one 16-token batch tile)")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_mma: act 0, or 1 (SwiGLU) with N % 16 == 0")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            check(self.lib.tw4_mma_persist(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), m, n, k, int(warps_k),
                                           int(unroll), int(ntile), int(per_cu), int(act), _stream(x)))
        return y

    def w4_mma_splitk(self, x, w, s, z, ws, locks, warps_k: int, unroll: int, ntile: int, splits: int,
                      act: int) -> torch.Tensor:
        """w4_mma with K split over `splits` workgroups per row-tile group (M <= 16): each covers
        1 / splits of the quant groups with x in LDS over that range; the last arriver adds the
        partial sums in split order (ws / locks: w4_gemm's workspace)."""
        m, n, k = check_operands("w4_mma", x, w, s, z)
        if not 1 <= m <= 16:
            raise RuntimeError("w4_mma_splitk: M <= 16 (one 16-token batch tile)")
        if not (ws.is_cuda and ws.dtype == torch.float32 and locks.is_cuda and locks.dtype == torch.int32
                and ws.device == x.device and locks.device == x.device and ws.is_contiguous()
                and locks.is_contiguous()):
            raise RuntimeError("w4_mma_splitk: float32 workspace and int32 locks (zero) on x's GPU")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_mma: act 0, or 1 (SwiGLU) with N % 16 == 0")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            check(self.lib.tw4_mma_splitk(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), _ptr(ws), _ptr(locks),
                                          ws.numel(), locks.numel(), m, n, k, int(warps_k), int(unroll), int(ntile),
                                          int(splits), int(act), _stream(x)))
        return y

    def w4_gemm(self, x, w, s, z, ws, locks, mt: int, nt: int, warps_n: int, warps_k: int, stages: int,
                splits: int, act: int) -> torch.Tensor:
        m, n, k = check_operands("w4_gemm", x, w, s, z)
        if not (ws.is_cuda and ws.dtype == torch.float32 and locks.is_cuda and locks.dtype == torch.int32
                and ws.device == x.device and locks.device == x.device and ws.is_contiguous()
                and locks.is_contiguous()):
            raise RuntimeError("w4_gemm: float32 workspace and int32 locks (zero) on x's GPU")
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_gemm: act 0, or 1 (SwiGLU) with N % 16 == 0")
        if m * k >= 1 << 31:
            raise RuntimeError("w4_gemm: M x K < 2^31")
        y = torch.empty((m, n // 2 if act else n), dtype=torch.float16, device=x.device)
        if m == 0:
            return y
        with torch.cuda.device(x.device):
            init_device(x.device)
            check(self.lib.tw4_gemm(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(y), _ptr(ws), _ptr(locks),
                                    ws.numel(), locks.numel(), m, n, k, int(mt), int(nt), int(warps_n),
                                    int(warps_k), int(stages), int(splits), int(act), _stream(x)))
        return y

    def w4_gemm_noalloc(self, x, w, s, z, mt: int, nt: int, warps_n: int, warps_k: int, stages: int, splits: int,
                        act: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """w4_gemm with the library's static split-K scratch instead of a workspace (tw4_gemm_noalloc: the
        C entry point allocates nothing). y comes from ``out`` (float16 [M, N] or [M, N / 2], contiguous,
        on x's GPU) or is allocated here with torch. Calls on one GPU share the scratch and must not
        overlap."""
        m, n, k = check_operands("w4_gemm_noalloc", x, w, s, z)
        if act not in (0, 1) or (act and n % 16):
            raise RuntimeError("w4_gemm_noalloc: act 0, or 1 (SwiGLU) with N % 16 == 0")
        if m * k >= 1 << 31:
            raise RuntimeError("w4_gemm_noalloc: M x K < 2^31")
        shape = (m, n // 2 if act else n)
        if out is None:
            out = torch.empty(shape, dtype=torch.float16, device=x.device)
        elif (tuple(out.shape) != shape or out.dtype != torch.float16 or out.device != x.device
              or not out.is_contiguous() or out.data_ptr() % 8):
            raise RuntimeError(f"w4_gemm_noalloc: out must be a contiguous float16 {list(shape)} tensor on x's GPU")
        if m == 0:
            return out
        with torch.cuda.device(x.device):
            init_device(x.device)
            check(self.lib.tw4_gemm_noalloc(_ptr(x), _ptr(w), _ptr(s), _ptr(z), _ptr(out), m, n, k, int(mt), int(nt),
                                            int(warps_n), int(warps_k), int(stages), int(splits), int(act),
                                            _stream(x)))
        return out

    def last_gemm_grid(self) -> tuple[int, int, int]:
        b, d, s = _I(), _I(), _I()
        self.lib.tw4_gemm_last_grid(ctypes.byref(b), ctypes.byref(d), ctypes.byref(s))
        return b.value, d.value, s.value


def repack(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
           interleave: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """AutoAWQ tensors (GPU) -> tile layout (packed [Npad, K/8] int32, scales [N, K/128] fp16,
    zeros [N, K/128] fp16) by the tw4_repack_awq kernel."""
    if not (qweight.is_cuda and qzeros.is_cuda and scales.is_cuda):
        raise RuntimeError("repack_awq: AutoAWQ tensors must be on the GPU (finalize after model.to(device))")
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32 or scales.dtype != torch.float16:
        raise RuntimeError("repack_awq: qweight / qzeros int32 and scales float16")
    k, n8 = qweight.shape
    n = 8 * n8
    if k % 128 or qzeros.shape != (k // 128, n8) or scales.shape != (k // 128, n):
        raise ValueError(f"repack_awq: qweight {tuple(qweight.shape)} qzeros {tuple(qzeros.shape)} "
                         f"scales {tuple(scales.shape)} group 128")
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    dev = qweight.device
    packed = torch.zeros((padded_rows(n), k // 8), dtype=torch.int32, device=dev)
    s_out = torch.empty((n, k // 128), dtype=torch.float16, device=dev)
    z_out = torch.empty((n, k // 128), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        check(library().tw4_repack_awq(_ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(packed), _ptr(s_out),
                                       _ptr(z_out), k, n, int(bool(interleave)), _stream(qweight)))
    return packed, s_out, z_out


def dequant(packed: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor, deinterleave: bool = False) -> torch.Tensor:
    """Tile layout -> dense fp16 [N, K] (bit-exact fp16_rne((q - z) s)) by the tw4_dequant kernel."""
    if not (packed.is_cuda and scales.is_cuda and zeros.is_cuda):
        raise RuntimeError("w4_dequant: tensors must be on the GPU")
    n, g = scales.shape
    k = 128 * g
    if (packed.dtype != torch.int32 or not packed.is_contiguous() or packed.shape != (padded_rows(n), k // 8)
            or scales.dtype != torch.float16 or zeros.dtype != torch.float16 or zeros.shape != scales.shape
            or not scales.is_contiguous() or not zeros.is_contiguous()):
        raise RuntimeError(f"w4_dequant: packed [{padded_rows(n)}, {k // 8}] int32 and contiguous float16 "
                           f"scales / zeros [N, K/128] (got {tuple(packed.shape)}, {tuple(scales.shape)})")
    out = torch.empty((n, k), dtype=torch.float16, device=packed.device)
    with torch.cuda.device(packed.device):
        check(library().tw4_dequant(_ptr(packed), _ptr(scales), _ptr(zeros), _ptr(out), n, k,
                                    int(bool(deinterleave)), _stream(packed)))
    return out


def read_probe(buf: torch.Tensor, sink: torch.Tensor, workgroups: int = 2048, chunked: bool = False,
               inflight: int = 1, key: int = 0x9E3779B9) -> None:
    """Read every byte of the contiguous GPU tensor ``buf`` once with 16-byte streaming loads and nothing
    else (tw4_read_probe), grid-stride or one contiguous span per workgroup (``chunked``), ``inflight``
    loads issued per lane before any is used, on the current stream: the plain-read ceiling of HBM. ``sink``: an int32 GPU tensor written only if the XOR of the
    data equals ``key``."""
    if not (buf.is_cuda and buf.is_contiguous() and buf.data_ptr() % 16 == 0 and (buf.numel() * buf.element_size()) % 16 == 0):
        raise RuntimeError("read_probe: a contiguous 16-byte aligned GPU tensor of a multiple of 16 bytes")
    if not (sink.is_cuda and sink.dtype == torch.int32 and sink.device == buf.device):
        raise RuntimeError("read_probe: sink must be an int32 tensor on the buffer's GPU")
    with torch.cuda.device(buf.device):
        check(library().tw4_read_probe(_ptr(buf), buf.numel() * buf.element_size(), int(workgroups), int(bool(chunked)),
                                       int(inflight), key & 0xFFFFFFFF, _ptr(sink), _stream(buf)))


def workspace(device: torch.device | str | int) -> tuple[torch.Tensor, torch.Tensor]:
    """w4_gemm's split-K buffers on a GPU: float32 partial sums and int32 counters, zero between
    calls (the kernel resets them). Allocated once, before graph capture; the GEMMs that use them
    must run on one stream at a time (w4_cuda.py:29-41)."""
    dev = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(index)
    if buf is None:
        dev = torch.device("cuda", index)
        buf = (torch.empty(WORKSPACE_FLOATS, dtype=torch.float32, device=dev),
               torch.zeros(WORKSPACE_LOCKS, dtype=torch.int32, device=dev))
        _workspaces[index] = buf
    return buf


@functools.lru_cache(maxsize=None)
def load() -> W4Extension | None:
    """The fused W4A16 kernels, or None when TANDEM_NO_CUDA_EXT=1 switches them off (the layer then
    dequantizes with the HIP kernel and multiplies with torch.matmul). Raises if the library is
    missing or no GPU is visible: there is no CPU path."""
    if os.environ.get("TANDEM_NO_CUDA_EXT") == "1":
        return None
    if not torch.cuda.is_available():
        raise RuntimeError("tandem_w4: no GPU visible (the W4A16 kernels run on MI355X / gfx950 only)")
    ext = W4Extension()
    init_device(torch.cuda.current_device())
    return ext
