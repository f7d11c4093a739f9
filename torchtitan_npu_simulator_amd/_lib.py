"""ctypes binding of the C ABI in ``include/dsa_mi355x.h``.

The HIP library is the only compute path: if it is not built, or no GPU is visible,
every op raises instead of falling back to anything else.
"""

from __future__ import annotations

import ctypes
import threading
import weakref
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libdsa_mi355x.so"
ABI_VERSION = 17

DSA_F32, DSA_BF16, DSA_FP8_E4M3 = 0, 1, 2

_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> argument types (must match include/dsa_mi355x.h)
_SIGNATURES = {
    "dsa_last_error": ([], ctypes.c_char_p),
    "dsa_abi_version": ([], _i32),
    "dsa_kernel_timing": ([_i32], _i32),
    "dsa_kernel_timing_count": ([], _i32),
    "dsa_kernel_timing_get": ([_i32, ctypes.c_char_p, _i64, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_int64)], _i32),
    "dsa_indexer_fwd": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp], _i32),
    "dsa_indexer_fwd_workspace_size": ([_i64, _i64, _i64, _i64, _i32], _i64),
    "dsa_indexer_fwd_ws": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                            _i64, _vp], _i32),
    "dsa_indexer_fwd_noalloc_max_rows": ([], _i64),
    "dsa_indexer_fwd_noalloc": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _vp], _i32),
    "dsa_quantize_fp8_rows": ([_vp, _i32, _vp, _vp, _i64, _i64, _vp], _i32),
    "dsa_attn_sink_fold": ([_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp], _i32),
    "dsa_attn_sink_grad": ([_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp], _i32),
    "dsa_topk": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp], _i32),
    "dsa_topk_workspace_size": ([_i64, _i64, _i64, _i64], _i64),
    "dsa_topk_ws": ([_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp], _i32),
    "dsa_lightning_indexer_workspace_size": ([_i64, _i64, _i64, _i64, _i64, _i32, _i64], _i64),
    "dsa_lightning_indexer": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                               _i64, _vp, _i64, _vp], _i32),
    "dsa_sparse_mla_fwd": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i64, _vp],
        _i32,
    ),
    "dsa_sparse_mla_bwd_workspace_size": ([_i64, _i64, _i64, _i64, _i64, _i64], _i64),
    "dsa_sparse_mla_bwd": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _f32, _i64, _vp],
        _i32,
    ),
    "dsa_sparse_mla_fwd_sink": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i64, _vp],
        _i32,
    ),
    "dsa_sparse_mla_bwd_sink": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _f32, _i64, _vp],
        _i32,
    ),
    "dsa_sparse_mla_bwd_ex": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _f32, _i64, _vp],
        _i32,
    ),
    "dsa_attn_mass": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _i64, _vp],
        _i32,
    ),
    "dsa_indexer_kl_grad_workspace_size": ([_i64, _i64, _i64, _i64, _i64, _i64], _i64),
    "dsa_indexer_kl_grad": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
         _f32, _f32, _vp, _vp],
        _i32,
    ),
    "dsa_indexer_kl_grad_ex": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _f32, _f32, _f32, _vp, _vp],
        _i32,
    ),
    "dsa_pair_csr_size": ([_i64, _i64, _i64, _i64], _i64),
    "dsa_sparse_mla_bwd_chunk_rows": ([_i64, _i64, _i64, _i64, _i64, _i64], _i64),
    "dsa_indexer_kl_grad_chunk_rows": ([_i64, _i64, _i64, _i64, _i64], _i64),
    "dsa_pair_csr_build": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp], _i32),
    "dsa_compressor_fwd": ([_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _f32, _vp, _i64, _i64, _vp,
                            _vp], _i32),
    "dsa_compressor_fwd_tnd": (
        [_vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _f32, _vp, _i64, _i64, _vp],
        _i32,
    ),
    "dsa_indexer_prep": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _i32, _vp],
                         _i32),
    "dsa_mla_absorb": ([_vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp], _i32),
    "dsa_tnd_metadata": ([_vp, _i32, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    # packed varlen: cu_seqlens / cmp_residual_k are host int32 arrays (ctypes arrays or None)
    "dsa_lightning_indexer_varlen": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp],
        _i32,
    ),
    "dsa_sparse_mla_fwd_varlen": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp],
        _i32,
    ),
    "dsa_sparse_mla_bwd_varlen_workspace_size": ([_vp, _vp, _i64, _i64, _i64, _i64], _i64),
    "dsa_sparse_mla_bwd_varlen": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
         _f32, _vp],
        _i32,
    ),
    "dsa_attn_mass_varlen": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp],
        _i32,
    ),
    # packed varlen with device cu_seqlens (device int32 pointers)
    "dsa_lightning_indexer_tnd_workspace_size": ([_i64, _i64, _i64, _i64, _i32, _i64, _i64], _i64),
    "dsa_lightning_indexer_tnd": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _vp, _i64, _vp],
        _i32,
    ),
    "dsa_tnd_global_indices": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp], _i32),
    "dsa_indexer_kl_grad_varlen_workspace_size": ([_vp, _vp, _i64, _i64, _i64, _i64], _i64),
    "dsa_indexer_kl_grad_varlen": (
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _f32, _f32,
         _vp, _vp],
        _i32,
    ),
}

_lib = None
_lock = threading.Lock()


class DSAError(RuntimeError):
    """Error reported by the HIP library (status code + dsa_last_error text)."""


def load_library(path: Path | None = None):
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise DSAError(
                f"HIP extension {p} is not built; run `python -m torchtitan_npu_simulator_amd.build` "
                "(there is no CPU fallback)"
            )
        lib = ctypes.CDLL(str(p))
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if lib.dsa_abi_version() != ABI_VERSION:
            raise DSAError(f"{p} has ABI {lib.dsa_abi_version()}, expected {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().dsa_last_error().decode(errors="replace")
        raise DSAError(f"{what} failed (status {rc}): {msg}")


class kernel_timing:
    """Context manager: HIP events around every kernel this library launches inside the
    block (dsa_kernel_timing).  ``summary()`` afterwards returns {kernel name: (total ms,
    launches)}, in the order the kernels first ran."""

    def __enter__(self):
        check(load_library().dsa_kernel_timing(1), "dsa_kernel_timing")
        self._summary = None
        return self

    def __exit__(self, *exc):
        check(load_library().dsa_kernel_timing(0), "dsa_kernel_timing")
        return False

    def summary(self) -> dict[str, tuple[float, int]]:
        if self._summary is None:
            lib = load_library()
            n = lib.dsa_kernel_timing_count()
            if n < 0:
                check(-n, "dsa_kernel_timing_count")
            out = {}
            buf = ctypes.create_string_buffer(256)
            ms, cnt = ctypes.c_double(), ctypes.c_int64()
            for i in range(n):
                check(lib.dsa_kernel_timing_get(i, buf, 256, ctypes.byref(ms), ctypes.byref(cnt)),
                      "dsa_kernel_timing_get")
                out[buf.value.decode()] = (ms.value, cnt.value)
            self._summary = out
        return self._summary


# host copies of device integer tensors (cu_seqlens and the like), keyed by the tensor and
# valid while its version counter is unchanged: the ops of one step that share a device
# cu_seqlens tensor read it back once, not once per op
# keyed by id(tensor): a WeakKeyDictionary would compare two weak references to the same
# live tensor with the tensor's own (elementwise) ==.  Each entry holds a weak reference,
# checked by identity, and is dropped when its tensor is freed.
_host_cache: dict[int, tuple["weakref.ref[torch.Tensor]", int, list[int]]] = {}


def _drop_host_entry(key: int, r: "weakref.ref[torch.Tensor]") -> None:
    entry = _host_cache.get(key)
    if entry is not None and entry[0] is r:  # (the id may have been reused since)
        del _host_cache[key]


def host_ints(values) -> list[int]:
    """``values`` (a list, a CPU tensor or a GPU tensor) as a host list of ints; a GPU
    tensor is read back once per version of that tensor."""
    if isinstance(values, torch.Tensor):
        if values.is_cuda:
            key = id(values)
            hit = _host_cache.get(key)
            if hit is not None and hit[0]() is values and hit[1] == values._version:
                return hit[2]
            lst = [int(v) for v in values.detach().to("cpu", torch.int64).tolist()]
            r = weakref.ref(values, lambda ref_, k=key: _drop_host_entry(k, ref_))
            _host_cache[key] = (r, values._version, lst)
            return lst
        return [int(v) for v in values.tolist()]
    return [int(v) for v in values]


def host_i32(values) -> ctypes.Array | None:
    """A host int32 array (ctypes) of ``values`` (a list or CPU/GPU tensor), or None."""
    if values is None:
        return None
    vals = host_ints(values)
    return (ctypes.c_int32 * len(vals))(*vals)


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of ``t`` for a kernel argument; a host tensor here would make the
    kernel dereference a CPU address, so it is refused."""
    if t is None:
        return None
    if not t.is_cuda:
        raise DSAError(f"a {tuple(t.shape)} {t.dtype} tensor on {t.device} was passed to a GPU kernel")
    return t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise DSAError(f"{name} must be a GPU tensor (the DSA ops have no CPU implementation)")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DSA_BF16
    if dt == torch.float32:
        return DSA_F32
    if dt == torch.float8_e4m3fn:
        return DSA_FP8_E4M3
    raise DSAError(f"unsupported dtype {dt}")
