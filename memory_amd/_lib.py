"""ctypes binding of libmoc.so (the C ABI declared in include/moc.h).

There is no CPU or PyTorch fallback: every op of this package runs the HIP
kernels of libmoc.so on a ROCm device and raises if the library is missing or
a tensor is not on the GPU.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libmoc.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "moc.h")

MOC_OK, MOC_ERR_ARG, MOC_ERR_UNSUPPORTED, MOC_ERR_LAUNCH = 0, 1, 2, 3
MOC_F32, MOC_BF16 = 0, 1
MOC_NORM_NONE, MOC_NORM_RMS, MOC_NORM_LAYERNORM = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGS = {
    "moc_last_error": (ctypes.c_char_p, []),
    "moc_abi_version": (_I, []),
    "moc_router_topk": (_I, [_P, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "moc_router_topk_bwd": (_I, [_P, _P, _P, _I64, _I64, _I, _I, _P, _P]),
    "moc_router_topk_bwd_pack_workspace": (_SZ, [_I64, _I64]),
    "moc_router_topk_bwd_pack": (_I, [_P, _P, _P, _I64, _I64, _I, _I, _P, _I64, _P, _P, _P, _SZ, _P]),
    "moc_prepend_shared": (_I, [_P, _P, _I64, _I, _I, _F, _P, _P, _P]),
    "moc_prepend_shared_bwd": (_I, [_P, _P, _I64, _I, _I, _F, _P, _P]),
    "moc_router_topk_prepend": (_I, [_P, _I64, _I64, _I, _I, _F, _P, _P, _P, _P, _P]),
    "moc_router_seq_bwd": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I, _I, _F, _P, _P, _P]),
    "moc_router_pool1": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "moc_seq_layer_saved_bytes": (_SZ, [_I64, _I64, _I64, _I, _I, _I64, _I, _I]),
    "moc_seq_layer_scratch_bytes": (_SZ, [_I64, _I64, _I64, _I, _I, _I64, _I, _I]),
    "moc_seq_layer_fwd": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _I64, _I, _I, _F,
                               _P, _P, _P, _P, _P, _P, _SZ, _P, _P]),
    "moc_seq_layer_bwd": (_I, [_P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _I, _I64, _I, _I, _F, _P, _P, _P, _P, _SZ,
                               _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I, _P, _P, _SZ, _P, _P, _P]),
    "moc_seq_layer_stage_count": (_I, []),
    "moc_seq_layer_stage_name": (ctypes.c_char_p, [_I]),
    "moc_seq_layer_timing": (_I, [ctypes.c_uint64, _I]),
    "moc_seq_layer_timing_read": (_I, [_P, _P, _P, _I]),
    "moc_rows_add_bcast": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _F, _P]),
    "moc_router_pool_workspace": (_SZ, [_I64, _I64, _I64]),
    "moc_router_pool": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "moc_router_linear": (_I, [_P, _I64, _I64, _P, _I, _P, _I64, _P, _P]),
    "moc_router_linear_bwd_workspace": (_SZ, [_I64, _I64, _I64]),
    "moc_router_linear_bwd": (_I, [_P, _P, _I64, _I64, _P, _I, _I64, _P, _P, _P, _P, _SZ, _P]),
    "moc_router_losses_workspace": (_SZ, [_I64, _I64]),
    "moc_router_losses": (_I, [_P, _I64, _I64, _P, _I, _P, _P, _P, _P, _P, _SZ, _P]),
    "moc_router_losses_bwd": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _P]),
    "moc_chapter_plan_workspace": (_SZ, [_I64, _I64]),
    "moc_chapter_plan": (_I, [_P, _I64, _I64, _P, _SZ, _P, _P, _P, _P, _P, _P]),
    "moc_chapter_plan_noalloc": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "moc_row_stats": (_I, [_P, _I, _I64, _I, _P, _P, _I64, _I, _F, _P, _P, _P]),
    "moc_kv_project": (_I, [_I, _P, _I, _I64, _I, _P, _P, _I64, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P]),
    "moc_chapter_project": (_I, [_P, _I64, _I, _P, _P, _I64, _P, _I, _I, _P, _I64, _P]),
    "moc_chapter_dx": (_I, [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I, _I, _I, _P, _I64, _I, _P]),
    "moc_weight_pack": (_I, [_P, _I, _P, _I, _I64, _I64, _P, _P, _P]),
    "moc_weight_transpose": (_I, [_P, _I, _I64, _I64, _P, _I64, _P]),
    "moc_dkv_multi_reduce": (_I, [_P, _I64, _P, _I64, _P, _P, _P, _P]),
    "moc_rows_linear": (_I, [_P, _I64, _I64, _P, _I, _I, _P, _I64, _P]),
    "moc_logit_grad_pack_workspace": (_SZ, [_I64, _I64]),
    "moc_logit_grad_pack": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "moc_rows_linear_residual": (_I, [_P, _I64, _I64, _P, _I, _I, _P, _I64, _P, _I64, _P]),
    "moc_rows_linear_f32": (_I, [_P, _I64, _I64, _P, _I, _I, _P, _P, _I64, _P]),
    "moc_norm_fold_weight": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "moc_rows_linear_norm": (_I, [_P, _I64, _I64, _P, _I, _I, _I, _F, _P, _P, _P, _I64, _P, _P, _P]),
    "moc_chapter_wgrad_workspace": (_SZ, [_I, _I, _I64]),
    "moc_chapter_wgrad": (_I, [_P, _I64, _P, _P, _I64, _I, _P, _P, _I64, _P, _P, _I, _I, _P, _SZ, _I, _P, _P]),
    "moc_xattn_fwd": (_I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _F, _P, _P,
                           _P]),
    "moc_xattn_weights": (_I, [_I, _P, _P, _I64, _I64, _I, _I, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _F, _P, _P,
                                _P]),
    "moc_xattn_bwd_prep": (_I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "moc_xattn_bwd_dq": (_I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I,
                              _I, _F, _P, _P]),
    "moc_xattn_bwd_dq_delta": (_I, [_I, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I,
                                    _I, _I, _I, _F, _P, _P]),
    "moc_xattn_bwd_dkv": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I,
                               _I, _F, _P, _P, _P]),
    "moc_kv_wgrad_workspace": (_SZ, [_I64, _I64, _I64]),
    "moc_kv_wgrad": (_I, [_P, _P, _I, _I64, _I, _P, _P, _P, _I64, _P, _P, _I64, _P, _SZ, _I, _P, _P]),
    "moc_linear_wgrad_workspace": (_SZ, [_I64, _I64, _I64]),
    "moc_linear_wgrad": (_I, [_P, _P, _I, _I64, _I64, _I64, _P, _SZ, _I, _P, _P]),
    "moc_dkv_reduce": (_I, [_I, _P, _P, _P, _P, _I64, _I64, _P, _P]),
    "moc_sparse_fwd": (_I, [_I, _P, _I64, _I, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _I64, _I, _I, _I,
                            _I, _I, _F, _P, _P, _P]),
    "moc_sparse_combine": (_I, [_I, _P, _P, _P, _P, _I, _I, _I, _I64, _I, _I, _P, _P, _P]),
    "moc_sparse_bwd_prep": (_I, [_I, _P, _P, _P, _P, _I, _I, _I, _I64, _I, _I, _P, _P]),
    "moc_sparse_bwd": (_I, [_I, _P, _P, _I64, _I, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _I64, _I, _I,
                            _I, _I, _I, _I, _P, _P, _P, _F, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "moc_sparse_dq_combine": (_I, [_I, _P, _P, _I, _I, _I64, _I, _I, _P, _P]),
    "moc_sparse_dw": (_I, [_P, _P, _P, _I, _I, _I64, _P, _P]),
    "moc_sparse_zero_untouched": (_I, [_I, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P, _P, _I64, _P, _P]),
    "moc_decode_partial": (_I, [_I, _P, _I64, _I, _P, _P, _I, _I, _I, _P, _P, _P, _P, _I64, _P, _I, _F, _P, _P, _P,
                                _P]),
    "moc_plan_row_table": (_I, [_P, _P, _P, _I64, _I, _P, _P]),
    "moc_decode_row_table": (_I, [_P, _P, _P, _I64, _P, _P]),
    "moc_gather_rows": (_I, [_I, _P, _I, _I64, _I, _P, _P, _I64, _P, _P, _P, _P]),
    "moc_bank_scatter": (_I, [_I, _P, _P, _I, _I64, _I, _P, _P, _I64, _P, _P, _P, _P, _I, _P, _P]),
    "moc_fill_zero": (_I, [_P, _I64, _I, _P]),
    "moc_bank_grad_accumulate": (_I, [_I, _P, _P, _I, _I64, _I, _P, _P, _I64, _P, _P, _P, _P, _I, _I, _P, _P, _P,
                                      _P]),
    "moc_bank_chunk_count": (_I, [_I64]),
    "moc_linear_rows": (_I, [_P, _I64, _I64, _P, _I64, _I, _P, _P]),
    "moc_row_norm_fwd": (_I, [_I, _I, _P, _I64, _I64, _P, _P, _F, _I, _P, _P, _P, _P]),
    "moc_row_norm_bwd_workspace": (_SZ, [_I64, _I64]),
    "moc_row_norm_bwd": (_I, [_I, _I, _P, _I64, _I64, _P, _P, _P, _I, _P, _I, _P, _P, _P, _SZ, _P]),
    "moc_bank_adamw": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I, _F, _F, _F, _F,
                            _F, _F, _P]),
    "moc_bank_touched": (_I, [_P, _I64, _I, _P, _P, _P]),
    "moc_bank_sqnorm_workspace": (_SZ, [_I64, _I64]),
    "moc_bank_sqnorm": (_I, [_P, _P, _P, _I64, _I64, _P, _SZ, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class MocError(RuntimeError):
    pass


def declared_symbols(header: str = HEADER):
    """Function names declared in include/moc.h."""
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moc_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load libmoc.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MocError(
                    f"libmoc.so not found at {LIB_PATH}; build it with `python -m memory_amd.build` "
                    "(memory_amd has no CPU fallback)")
            l = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                f = getattr(l, name)
                f.restype = res
                f.argtypes = args
            _lib = l
    return _lib


# Optional per-entry-point GPU timing: when set to a dict, every call records a
# pair of events on the current stream (the one the kernels are launched on),
# appended to KERNEL_EVENTS[name]; KERNEL_EVENTS_ONLY (a set of names) limits the
# recording to those entry points.
KERNEL_EVENTS = None
KERNEL_EVENTS_ONLY = None


def call(name: str, *args) -> None:
    ev = KERNEL_EVENTS
    if ev is not None and (KERNEL_EVENTS_ONLY is None or name in KERNEL_EVENTS_ONLY):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = getattr(lib(), name)(*args)
        e1.record()
        ev.setdefault(name, []).append((e0, e1))
    else:
        rc = getattr(lib(), name)(*args)
    if rc != MOC_OK:
        msg = lib().moc_last_error().decode(errors="replace")
        if rc in (MOC_ERR_ARG, MOC_ERR_UNSUPPORTED):
            raise ValueError(f"{name}: {msg}")
        raise MocError(f"{name} failed ({rc}): {msg}")


def seq_stage_names():
    """Names of the timed stages of moc_seq_layer_fwd / _bwd, in stage order."""
    l = lib()
    return [l.moc_seq_layer_stage_name(i).decode() for i in range(l.moc_seq_layer_stage_count())]


def seq_stage_timing(names=None, capacity: int = 0) -> None:
    """Arm timing events around the next ``capacity`` launches of the named stages of the
    native layer (all stages when ``names`` is None; ``capacity`` 0 disarms)."""
    all_names = seq_stage_names()
    want = set(all_names) if names is None else set(names)
    unknown = want - set(all_names)
    if unknown:
        raise ValueError(f"unknown moc_seq_layer stages: {sorted(unknown)}")
    mask = sum(1 << i for i, n in enumerate(all_names) if n in want) if capacity else 0
    call("moc_seq_layer_timing", ctypes.c_uint64(mask), int(capacity))


def seq_stage_read():
    """{stage name: (summed ms, timed launches, launches past capacity)} for the stages that ran
    since arming; clears the counts (the stages stay armed)."""
    names = seq_stage_names()
    n = len(names)
    tot = (ctypes.c_double * n)()
    cnt = (ctypes.c_int32 * n)()
    drop = (ctypes.c_int32 * n)()
    call("moc_seq_layer_timing_read", ctypes.cast(tot, _P), ctypes.cast(cnt, _P), ctypes.cast(drop, _P), n)
    return {names[i]: (tot[i], cnt[i], drop[i]) for i in range(n) if cnt[i] or drop[i]}


class region:
    """``with region(name): ...`` records a pair of events around work that is not a libmoc
    entry point (a library GEMM, a torch op) under the same rules as ``call``, so that the
    per-kernel table accounts for the whole step."""

    def __init__(self, name: str):
        self.name = name
        self.ev = None

    def __enter__(self):
        ev = KERNEL_EVENTS
        if ev is not None and (KERNEL_EVENTS_ONLY is None or self.name in KERNEL_EVENTS_ONLY):
            self.ev = ev
            self.e0 = torch.cuda.Event(enable_timing=True)
            self.e0.record()
        return self

    def __exit__(self, *exc):
        if self.ev is not None:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record()
            self.ev.setdefault(self.name, []).append((self.e0, e1))
        return False


def query(name: str, *args):
    return getattr(lib(), name)(*args)


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MOC_F32
    if dt == torch.bfloat16:
        return MOC_BF16
    raise ValueError(f"memory_amd kernels support float32 and bfloat16 tensors, got {dt}")


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "memory_amd runs only on ROCm devices (HIP kernels of libmoc.so); got a tensor on "
                f"{t.device}. There is no CPU fallback.")
