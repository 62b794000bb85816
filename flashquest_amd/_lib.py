"""ctypes binding of libfq_hip.so (the C ABI declared in include/fq_hip.h).

The HIP library is the only compute path: every operator in this package
calls into it, and a missing or unloadable library raises instead of falling
back to anything else.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

# FQ_HIP_LIBRARY selects another build of the same library (e.g. a debug build).
LIB_PATH = os.environ.get("FQ_HIP_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib",
                                                            "libfq_hip.so")

FQ_OK, FQ_ERR_INVALID, FQ_ERR_UNSUPPORTED, FQ_ERR_HIP, FQ_ERR_WORKSPACE = range(5)
FQ_BF16, FQ_F16, FQ_F32 = 0, 1, 2
FQ_SELECT_PER_Q_HEAD, FQ_SELECT_PER_KV_HEAD_SUM = 0, 1

SELECT_MODES = {"per_q_head": FQ_SELECT_PER_Q_HEAD, "per_kv_head_sum": FQ_SELECT_PER_KV_HEAD_SUM}

_I64x3 = ctypes.c_int64 * 3
_I64x4 = ctypes.c_int64 * 4
_I64x5 = ctypes.c_int64 * 5
I64x5 = _I64x5
I64x4 = _I64x4
I64x3 = _I64x3


class Int4Cache(ctypes.Structure):
    _fields_ = [
        ("k_packed", ctypes.c_void_p), ("k_strides", _I64x5),
        ("v_packed", ctypes.c_void_p), ("v_strides", _I64x5),
        ("k_scale", ctypes.c_void_p), ("ks_strides", _I64x5),
        ("k_mn", ctypes.c_void_p), ("km_strides", _I64x5),
        ("v_scale", ctypes.c_void_p), ("vs_strides", _I64x5),
        ("v_mn", ctypes.c_void_p), ("vm_strides", _I64x5),
        ("meta_dtype", ctypes.c_int32),
        ("L", ctypes.c_int32), ("B", ctypes.c_int32), ("H_kv", ctypes.c_int32),
        ("S", ctypes.c_int32), ("P", ctypes.c_int32), ("D", ctypes.c_int32),
        ("page_size", ctypes.c_int32), ("v_groups", ctypes.c_int32),
    ]


class Query(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_dtype", ctypes.c_int32), ("q_strides", _I64x4),
        ("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int32), ("o_strides", _I64x4),
        ("lse", ctypes.c_void_p), ("lse_strides", _I64x3),
        ("H_q", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("retention_layer_stride", ctypes.c_int64), ("rotation_signs", ctypes.c_void_p),
    ]


class Tail(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p), ("k_strides", _I64x5),
        ("v", ctypes.c_void_p), ("v_strides", _I64x5),
        ("dtype", ctypes.c_int32), ("len", ctypes.c_int32), ("D", ctypes.c_int32),
    ]


class Prefill(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_strides", _I64x4),
        ("out", ctypes.c_void_p), ("o_strides", _I64x4),
        ("H_q", ctypes.c_int32), ("S_q", ctypes.c_int32),
        ("causal_offset", ctypes.c_int32), ("sm_scale", ctypes.c_float),
        ("D", ctypes.c_int32),
    ]


class TurboCache(ctypes.Structure):
    _fields_ = [
        ("k_msb", ctypes.c_void_p), ("kmsb_strides", _I64x5),
        ("k_lsb", ctypes.c_void_p), ("klsb_strides", _I64x5),
        ("k_scale", ctypes.c_void_p), ("kst_strides", _I64x5),
        ("v_msb", ctypes.c_void_p), ("vmsb_strides", _I64x5),
        ("v_lsb", ctypes.c_void_p), ("vlsb_strides", _I64x5),
        ("v_scale", ctypes.c_void_p), ("vst_strides", _I64x5),
        ("L", ctypes.c_int32), ("B", ctypes.c_int32), ("H_kv", ctypes.c_int32),
        ("S", ctypes.c_int32), ("P", ctypes.c_int32), ("D", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int32
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); the list every test checks the export table against
SIGNATURES = {
    "fq_last_error": (ctypes.c_char_p, []),
    "fq_abi_version": (ctypes.c_int, []),
    "fq_kernel_timer_start": (ctypes.c_int, [_I]),
    "fq_set_attention_splits": (ctypes.c_int, [_I]),
    "fq_kernel_timer_stop": (ctypes.c_int, [ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int32)]),
    "fq_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Int4Cache), _I]),
    "fq_turbo_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(TurboCache), _I]),
    "fq_page_scores_int4": (ctypes.c_int, [_P, _I, _I64P, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                           _I, _I, _I, _I, _I, _I, _P]),
    "fq_select_pages": (ctypes.c_int, [_P, _I64P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I64P, _P]),
    "fq_compact_ids": (ctypes.c_int, [_P, _I64P, _I, _I, _I, _I, _I, _P, _P]),
    "fq_sparse_int4_fwd_mask": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I64P,
                                               _P, ctypes.c_size_t, _P]),
    "fq_sparse_int4_fwd_ids": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I64P, _I,
                                              _P, ctypes.c_size_t, _P]),
    "fq_quest_decode_int4": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I, _I, _I,
                                            _P, _P, _P, ctypes.c_size_t, _P]),
    "fq_quest_decode_int4_noalloc": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I,
                                                    _I, _I, _P, _P, _P]),
    "fq_quest_select_int4": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I, _I, _I,
                                            _P, _P, _P, ctypes.c_size_t, _P]),
    "fq_int4_cache_append": (ctypes.c_int, [ctypes.POINTER(Int4Cache), _I, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                            _P, _I64P, _I, _I, _P]),
    "fq_int8_cache_append": (ctypes.c_int, [ctypes.POINTER(Int4Cache), _I, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                            _P, _I64P, _I, _I, _P]),
    "fq_turbo_cache_append": (ctypes.c_int, [ctypes.POINTER(TurboCache), _P, _I64P, _P, _I64P, _I, _P, _I64P, _P,
                                             _I64P, _I, _P, _I64P, _P, _I64P, _I, _I, _P]),
    "fq_quest_decode_turbo": (ctypes.c_int, [ctypes.POINTER(TurboCache), _P, _I64P, _P, _I64P, ctypes.POINTER(Query),
                                             _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t, _P]),
    "fq_quest_select_turbo": (ctypes.c_int, [ctypes.POINTER(TurboCache), _P, _I64P, _P, _I64P, ctypes.POINTER(Query),
                                             _P, _I, _I, _I, _I, _P, _P, ctypes.c_size_t, _P]),
    "fq_quest_decode_int4_tail": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), ctypes.POINTER(Tail),
                                                 _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "fq_quest_decode_int8_tail": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), ctypes.POINTER(Tail),
                                                 _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P]),
    "fq_quest_fused_int4": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _I, _I, _I, _I]),
    "fq_quest_fused_int8": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _I, _I, _I, _I]),
    "fq_quest_fused_turbo": (ctypes.c_int, [ctypes.POINTER(TurboCache), ctypes.POINTER(Query)]),
    "fq_quest_attend_int4": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I, _I, _I,
                                            _P, ctypes.c_size_t, _P]),
    "fq_merge_attn": (ctypes.c_int, [_P, _P, _P, _P, _I, ctypes.c_int64, ctypes.c_int64, _P, ctypes.c_int64, _P,
                                     _I, _I, _P]),
    "fq_dense_tail_attn": (ctypes.c_int, [_P, _I64P, _P, _I64P, _P, _I64P, _I, _P, _I64P, _P,
                                          _I, _I, _I, _I, _I, _P]),
    "fq_quantize_k_int4": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _I, _P, _I64P, _P, _I64P, _P, _I64P,
                                          _I, _P]),
    "fq_quantize_v_int4": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _I, _P, _I64P, _P, _I64P, _P, _I64P,
                                          _I, _P]),
    "fq_wht": (ctypes.c_int, [_P, _I, ctypes.c_int64, _P, _I, ctypes.c_int64, _I, _I, _P, _I, _I, _P]),
    "fq_quantize_turbo": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _P, _I64P, _P, _I64P, _P, _I64P, _P]),
    "fq_sparse_turbo_fwd_mask": (ctypes.c_int, [ctypes.POINTER(TurboCache), ctypes.POINTER(Query), _P, _I64P,
                                                _P, ctypes.c_size_t, _P]),
    # INT8 family (fq_int8_cache has the fq_int4_cache layout)
    "fq_int8_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Int4Cache), _I]),
    "fq_page_scores_int8": (ctypes.c_int, [_P, _I, _I64P, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                           _I, _I, _I, _I, _I, _I, _P]),
    "fq_page_scores_int8_summary": (ctypes.c_int, [_P, _I, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _I, _P, _P,
                                                   _I64P, _P, _I64P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "fq_page_summary": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _I, _P, _P, _I64P, _P]),
    "fq_page_scores_quest": (ctypes.c_int, [_P, _I, _I64P, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                            _I, _I, _I, _I, _I, _I, _P]),
    "fq_page_scores_int8_bound": (ctypes.c_int, [_P, _I, _I64P, _P, _I64P, _P, _I64P, _I, _P, _I64P,
                                                 _I, _I, _I, _I, _I, _I, _P]),
    "fq_sparse_int8_fwd_mask": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I64P,
                                               _P, ctypes.c_size_t, _P]),
    "fq_quest_decode_int8": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I, _I, _I,
                                            _P, _P, _P, ctypes.c_size_t, _P]),
    "fq_quest_select_int8": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Query), _P, _I, _I, _I, _I,
                                            _P, _P, _P, ctypes.c_size_t, _P]),
    "fq_quantize_k_int8": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _I, _P, _I64P, _P, _I64P, _P, _I64P,
                                          _I, _P]),
    "fq_quantize_v_int8": (ctypes.c_int, [_P, _I, _I64P, _I, _I, _I, _I, _P, _I64P, _P, _I64P, _P, _I64P,
                                          _I, _P]),
    # prefill over the packed cache
    "fq_prefill_int4": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Tail), ctypes.POINTER(Prefill),
                                       _P, ctypes.c_size_t, _P]),
    "fq_prefill_int8": (ctypes.c_int, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Tail), ctypes.POINTER(Prefill),
                                       _P, ctypes.c_size_t, _P]),
    "fq_prefill_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Int4Cache), ctypes.POINTER(Tail),
                                                     ctypes.POINTER(Prefill), _I]),
    "fq_prefill_turbo": (ctypes.c_int, [ctypes.POINTER(TurboCache), ctypes.POINTER(Tail), ctypes.POINTER(Prefill),
                                        _P, ctypes.c_size_t, _P]),
    "fq_prefill_turbo_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(TurboCache), ctypes.POINTER(Tail),
                                                           ctypes.POINTER(Prefill)]),
}

_lib = None
_lock = threading.Lock()


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libfq_hip.so once; raises RuntimeError when it is missing."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"libfq_hip.so not found at {path}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or `python -m flashquest_amd.build`")
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load_library()


def check(status: int, what: str = "") -> None:
    """Map an fq_status to the reference's exception types."""
    if status == FQ_OK:
        return
    msg = lib().fq_last_error().decode(errors="replace")
    msg = f"{what}: {msg}" if what else msg
    if status == FQ_ERR_INVALID:
        raise ValueError(msg)
    if status == FQ_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


_DTYPES = {torch.bfloat16: FQ_BF16, torch.float16: FQ_F16, torch.float32: FQ_F32}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise AssertionError(f"unsupported dtype {dt}") from None


def i64(values, n: int):
    vals = list(values)
    if len(vals) != n:
        raise ValueError(f"expected {n} strides, got {len(vals)}")
    return (ctypes.c_int64 * n)(*vals)


_I64_ARRAYS = {n: ctypes.c_int64 * n for n in range(1, 9)}


def strides(t: torch.Tensor, n: int | None = None, lead: int = 0):
    """Element strides of t, left-padded with `lead` zeros (broadcast axes)."""
    st = t.stride()
    if n is None:
        n = lead + len(st)
    elif lead + len(st) != n:
        raise ValueError(f"expected {n} strides, got {lead + len(st)}")
    return _I64_ARRAYS[n](*((0,) * lead + st))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device | None = None) -> int:
    """The raw HIP stream torch currently launches on for `device`."""
    idx = device.index if isinstance(device, torch.device) else device
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise AssertionError("flashquest_amd operators need ROCm device tensors (HIP path only)")


# ---------------------------------------------------------------- workspace --
_ws: dict = {}


def workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Per-(device, stream) scratch buffer, zero-initialised when (re)allocated.

    Every region a call reads (selection lists, counts, split partials) is
    written earlier in the same call, so the buffer is reused across calls
    without clearing.  Calls that overlap on one stream are serialised by the
    stream; distinct streams get distinct buffers.
    """
    key = (device.index, stream_handle(device) if stream is None else stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("workspace must be allocated before HIP graph capture (run once eagerly)")
        buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _ws[key] = buf
    return buf


class KernelTimer:
    """Times the sparse-attention kernels launched from this thread (HIP events
    around each launch, recorded by the library on the launch stream)."""

    def __init__(self, max_launches: int):
        self.max_launches = int(max_launches)

    def __enter__(self):
        check(lib().fq_kernel_timer_start(self.max_launches), "kernel timer")
        return self

    def __exit__(self, *exc):
        ms, n = ctypes.c_float(0.0), ctypes.c_int32(0)
        check(lib().fq_kernel_timer_stop(ctypes.byref(ms), ctypes.byref(n)), "kernel timer")
        self.total_ms, self.launches = ms.value, n.value
        return False


class attention_splits:
    """Context manager: fixed workgroups per KV group for the matrix-core INT4
    attention kernel (tests and tuning); restores the automatic choice on exit."""

    def __init__(self, splits: int):
        self.splits = int(splits)

    def __enter__(self):
        check(lib().fq_set_attention_splits(self.splits), "attention splits")
        return self

    def __exit__(self, *exc):
        check(lib().fq_set_attention_splits(0), "attention splits")
        return False
