"""The benchmark's measurement probes (libfq_probe.so, declared in
flashquest_amd/csrc/fq_probe.h): reads with the decode step's access pattern
that compute nothing.  Not part of the product library or its C ABI; only
bench.py and the tests that cover the bench use them."""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from . import _lib as L
from ._ops import int4_cache

PROBE_PATH = os.path.join(os.path.dirname(L.LIB_PATH), "libfq_probe.so")
SIGNATURES = {
    "fq_read_decode_pages": (ctypes.c_int, [ctypes.POINTER(L.Int4Cache), L._P, L._I64P, L._I, L._P, L._P,
                                            ctypes.c_size_t, L._P]),
    "fq_read_stream": (ctypes.c_int, [L._P, ctypes.c_size_t, L._P, L._P]),
}
_probe = None
_lock = threading.Lock()


def probe_lib() -> ctypes.CDLL:
    """Load libfq_probe.so (after libfq_hip.so, whose helpers it uses)."""
    global _probe
    with _lock:
        if _probe is None:
            L.lib()
            if not os.path.exists(PROBE_PATH):
                raise RuntimeError(f"libfq_probe.so not found at {PROBE_PATH}; build with `python -m flashquest_amd.build`")
            lib = ctypes.CDLL(PROBE_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _probe = lib
    return _probe


def read_decode_pages(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, mask: torch.Tensor,
                      page_size: int = 64) -> None:
    """Measurement only (no counterpart in the reference): read exactly the
    bytes a single-launch INT4 decode step reads for the selection ``mask``
    (L, B, H_q, P), in the same order, and compute nothing.  Its time is the
    memory system's ceiling for the step's access pattern."""
    c, keep = int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size)
    L.require_device(mask, *keep)
    if mask.dtype != torch.bool or mask.dim() != 4:
        raise ValueError(f"mask must be a 4D (L, B, H_q, P) bool tensor, got {mask.dtype} {tuple(mask.shape)}")
    H_q = mask.shape[2]
    if (mask.shape[0], mask.shape[1], mask.shape[3]) != (c.L, c.B, c.P):
        raise ValueError(f"mask {tuple(mask.shape)} does not match the cache's (L={c.L}, B={c.B}, H_q, P={c.P})")
    ws = L.workspace(mask.device, L.lib().fq_workspace_bytes(c, H_q))
    sink = torch.zeros(1, dtype=torch.int32, device=mask.device)
    L.check(probe_lib().fq_read_decode_pages(c, mask.data_ptr(), L.strides(mask, 4), H_q, sink.data_ptr(),
                                         ws.data_ptr(), ws.numel(), L.stream_handle(mask.device)),
            "read_decode_pages")


def read_stream(buf: torch.Tensor) -> None:
    """Measurement only (no counterpart in the reference): read the bytes of
    the contiguous device tensor ``buf`` with plain streaming loads and compute
    nothing -- the HBM read rate for that byte count with no access pattern."""
    L.require_device(buf)
    if not buf.is_contiguous():
        raise ValueError("read_stream takes a contiguous tensor")
    sink = torch.zeros(1, dtype=torch.int32, device=buf.device)
    nbytes = buf.numel() * buf.element_size()
    L.check(probe_lib().fq_read_stream(buf.data_ptr(), nbytes, sink.data_ptr(), L.stream_handle(buf.device)), "read_stream")
