"""Tensor -> C-ABI descriptor plumbing shared by the operator modules."""
from __future__ import annotations

import math

import torch

from . import _lib as L


def _ensure_inner_contiguous(t: torch.Tensor, align_elems: int = 1) -> torch.Tensor:
    """Kernels need a unit-stride innermost axis and aligned rows; copy otherwise."""
    st = t.stride()
    ok = st[-1] == 1
    if ok and align_elems > 1:
        for s in st[:-1]:
            if s % align_elems:
                ok = False
                break
        ok = ok and t.data_ptr() % (align_elems * t.element_size()) == 0
    if not ok:
        # a fresh copy: contiguous() would return a contiguous but misaligned view unchanged
        return t.clone(memory_format=torch.contiguous_format)
    return t


def _lead(t: torch.Tensor, want: int) -> int:
    if t.dim() not in (want - 1, want):
        raise ValueError(f"expected a {want - 1}D or {want}D tensor, got {tuple(t.shape)}")
    return want - t.dim()


def int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size: int):
    """Describe a packed INT4 cache view: 4D (B,H,S,X) per layer or 5D (L,B,H,S,X).

    Returns (descriptor, keepalive tensors).
    """
    kp = _ensure_inner_contiguous(K_packed, 4)
    vp = _ensure_inner_contiguous(V_packed, 4)
    ks = _ensure_inner_contiguous(K_scale, 8)
    km = _ensure_inner_contiguous(K_mn, 8)
    vs = _ensure_inner_contiguous(V_scale)
    vm = _ensure_inner_contiguous(V_mn)
    if ks.dtype != km.dtype or vs.dtype != ks.dtype or vm.dtype != ks.dtype:
        raise AssertionError("K_scale, K_mn, V_scale and V_mn must share one dtype")
    if ks.dtype not in (torch.bfloat16, torch.float16):
        raise AssertionError(f"metadata dtype must be bf16 or fp16, got {ks.dtype}")
    lead = _lead(kp, 5)
    nd = kp.dim()
    if vp.dim() != nd or ks.dim() != nd or km.dim() != nd or vs.dim() != nd or vm.dim() != nd:
        raise ValueError("the six cache tensors must have the same number of dimensions")
    pad = (0,) * lead
    a5 = L.I64x5
    shape = (1,) * lead + tuple(kp.shape)
    c = L.Int4Cache(kp.data_ptr(), a5(*(pad + kp.stride())), vp.data_ptr(), a5(*(pad + vp.stride())),
                    ks.data_ptr(), a5(*(pad + ks.stride())), km.data_ptr(), a5(*(pad + km.stride())),
                    vs.data_ptr(), a5(*(pad + vs.stride())), vm.data_ptr(), a5(*(pad + vm.stride())),
                    L.dtype_code(ks.dtype), shape[0], shape[1], shape[2], shape[3], ks.shape[-2],
                    shape[4] * 2, int(page_size), vs.shape[-1])
    return c, (kp, vp, ks, km, vs, vm)


def int8_cache(K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, page_size: int):
    """Describe an INT8 cache view (one code byte per channel; V metadata per
    token): 4D (B,H,S,D) per layer or 5D (L,B,H,S,D).  Same descriptor layout
    as the INT4 one.  Returns (descriptor, keepalive tensors)."""
    ku = _ensure_inner_contiguous(K_uint8, 8)
    vu = _ensure_inner_contiguous(V_uint8, 8)
    c, keep = int4_cache(ku, K_scale, K_mn, vu, V_scale, V_mn, page_size)
    c.D = ku.shape[-1]
    if c.v_groups != 1:
        raise AssertionError("INT8 V metadata must be per token: (..., S, 1)")
    return c, keep


def turbo_cache(K_msb, K_lsb, K_scale, V_msb, V_lsb, V_scale, num_pages: int, page_size: int):
    D = K_msb.shape[-1] * 8
    if (V_msb.shape[-1] * 8, K_lsb.shape[-1] * 4, V_lsb.shape[-1] * 4) != (D, D, D):
        raise AssertionError(f"TurboQuant planes disagree on head_dim: MSB rows {K_msb.shape[-1]}/{V_msb.shape[-1]} "
                             f"bytes (D/8), LSB rows {K_lsb.shape[-1]}/{V_lsb.shape[-1]} bytes (D/4)")
    if K_scale.shape[-1] != 1 or V_scale.shape[-1] != 1:
        raise AssertionError("TurboQuant scales must be per token: (..., S, 1)")
    ts = [_ensure_inner_contiguous(t) for t in (K_msb, K_lsb, K_scale, V_msb, V_lsb, V_scale)]
    lead = _lead(ts[0], 5)
    c = L.TurboCache()
    c.k_msb, c.kmsb_strides = ts[0].data_ptr(), L.strides(ts[0], 5, lead)
    c.k_lsb, c.klsb_strides = ts[1].data_ptr(), L.strides(ts[1], 5, lead)
    c.k_scale, c.kst_strides = ts[2].data_ptr(), L.strides(ts[2], 5, lead)
    c.v_msb, c.vmsb_strides = ts[3].data_ptr(), L.strides(ts[3], 5, lead)
    c.v_lsb, c.vlsb_strides = ts[4].data_ptr(), L.strides(ts[4], 5, lead)
    c.v_scale, c.vst_strides = ts[5].data_ptr(), L.strides(ts[5], 5, lead)
    shape = (1,) * lead + tuple(ts[0].shape)
    c.L, c.B, c.H_kv, c.S = shape[0], shape[1], shape[2], shape[3]
    if num_pages > -(-c.S // page_size):
        raise ValueError(f"TurboQuant cache: {num_pages} pages but the planes hold {c.S} tokens "
                         f"({-(-c.S // page_size)} pages of {page_size})")
    c.D = ts[0].shape[-1] * 8
    c.P = int(num_pages)
    c.page_size = int(page_size)
    return c, ts


def query(Q3: torch.Tensor, O3: torch.Tensor, lse: torch.Tensor | None, sm_scale: float | None):
    """Q3/O3: (B, H_q, D) or (L, B, H_q, D); lse: (B, H_q) / (L, B, H_q) or None."""
    lead = 4 - Q3.dim()
    pad = (0,) * lead
    if O3.dim() != Q3.dim() or (lse is not None and lse.dim() != Q3.dim() - 1):
        raise ValueError("query, output and lse ranks disagree")
    D = Q3.shape[-1]
    return L.Query(Q3.data_ptr(), L.dtype_code(Q3.dtype), L.I64x4(*(pad + Q3.stride())),
                   O3.data_ptr(), L.dtype_code(O3.dtype), L.I64x4(*(pad + O3.stride())),
                   None if lse is None else lse.data_ptr(),
                   L.I64x3(*(pad + lse.stride())) if lse is not None else L.I64x3(0, 0, 0),
                   Q3.shape[-2], float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(D), 0, None)


def retention_rows(retention, head_pattern, H_q: int, H_kv: int, layers: int, device):
    """The retention array of a decode call and its layer stride.

    Without ``head_pattern``: retention_tensor's (H_q,) vector, stride 0.
    With ``head_pattern`` (H_kv,) or (layers, H_kv) bool (True = retrieval,
    False = streaming): query heads of streaming KV heads get retention 0, so
    they keep only the sink and window pages, the others the given retention
    (llama_persistent_patch.py:214-220, duo/fused_dispatch.py:56-62).  A
    per-layer pattern gives an (layers, H_q) array with stride H_q.
    """
    r = retention_tensor(retention, H_q, device)
    if head_pattern is None:
        return r, 0
    pat = torch.as_tensor(head_pattern)
    if pat.dtype != torch.bool:
        raise ValueError(f"head_pattern must be a bool tensor; got {pat.dtype}")
    if pat.shape not in ((H_kv,), (layers, H_kv)):
        raise ValueError(f"head_pattern must be ({H_kv},) or ({layers}, {H_kv}) (KV heads, per layer); "
                         f"got {tuple(pat.shape)}")
    per_q = pat.to(device).repeat_interleave(H_q // H_kv, dim=-1)
    rows = torch.where(per_q, r, torch.zeros_like(r)).contiguous()
    return rows, (H_q if rows.dim() == 2 else 0)


# Device (H,) vectors of scalar retentions, made once per (value, H, device):
# a decode step per layer would otherwise launch a fill kernel every call.
# The kernels only read them.
_scalar_retention: dict = {}


def retention_tensor(retention, H: int, device) -> torch.Tensor:
    """selection.py:92-101: scalar in [0, 1] or a (H,) tensor -> device fp32 (H,)."""
    if isinstance(retention, torch.Tensor):
        if retention.shape != (H,):
            raise ValueError(f"per-head retention must be shape ({H},); got {tuple(retention.shape)}")
        # the kernels read H contiguous floats: a strided view is copied
        return retention.to(device=device, dtype=torch.float32).contiguous()
    if not (0.0 <= float(retention) <= 1.0):
        raise ValueError(f"scalar retention must be in [0, 1]; got {retention}")
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (float(retention), H, device.type, device.index)
    r = _scalar_retention.get(key)
    if r is None:
        r = torch.full((H,), float(retention), dtype=torch.float32, device=device)
        # a tensor made during HIP graph capture lives in the graph's pool: not kept
        if not (device.type == "cuda" and torch.cuda.is_current_stream_capturing()):
            if len(_scalar_retention) >= 256:       # callers that vary the retention every step
                # kernels queued on any stream may still read the cached
                # vectors: let every one of them finish before the memory can
                # be reused
                for d in {k[3] for k in _scalar_retention if k[2] == "cuda"}:
                    torch.cuda.synchronize(d)
                _scalar_retention.clear()
            if device.type == "cuda":
                # shared by calls on every stream: the fill must be done before any reads it
                torch.cuda.current_stream(device).synchronize()
            _scalar_retention[key] = r
    return r


# ---- GQA ratios above 4 on the matrix-core kernels ---------------------------
# Those kernels take at most 4 query heads per KV head.  The fused decode
# entries run 6 or 8 as virtual KV heads themselves where the attention kernel
# selects its own pages; every other group of more than 4 is attended here in
# chunks of its query heads, each chunk reading the group's pages.

def head_chunks(nrep: int):
    """(offset, size) chunks of a KV group's query heads, each of at most 4
    heads, sizes as equal as possible (8 -> 4 + 4, 7 -> 4 + 3, 5 -> 3 + 2)."""
    n = -(-nrep // 4)
    base, extra = divmod(nrep, n)
    chunks, off = [], 0
    for i in range(n):
        size = base + (1 if i < extra else 0)
        chunks.append((off, size))
        off += size
    return chunks


def heads(x, axis: int, H_kv: int, nrep: int, off: int, size: int):
    """The query heads [off, off + size) of every KV group of x's head axis
    `axis` (H_kv * nrep heads, group-major), as a contiguous tensor."""
    return x.unflatten(axis, (H_kv, nrep)).narrow(axis + 1, off, size).flatten(axis, axis + 1).contiguous()


def put_heads(dst, src, axis: int, H_kv: int, nrep: int, off: int, size: int):
    """Writes src (H_kv * size heads on `axis`) back into those heads of dst."""
    dst.unflatten(axis, (H_kv, nrep)).narrow(axis + 1, off, size).copy_(src.unflatten(axis, (H_kv, size)))


def wants_head_chunks(H_q: int, H_kv: int, D: int, page_size: int) -> bool:
    """5 to 8 query heads per KV head on the matrix-core layout (head_dim 128,
    64-token pages), and more than 8 on any layout (the library's kernels take
    at most 8: one selection bit per query head of a group): chunked, unless
    the decode entry takes 6 or 8 on virtual KV heads itself (the callers ask
    the library).  Other shapes take their kernels whole."""
    if H_kv < 1 or H_q % H_kv:
        return False
    nrep = H_q // H_kv
    return nrep > 8 or (nrep > 4 and D == 128 and page_size == 64)


def attend_in_head_chunks(Q, H_kv: int, per_head, call, return_lse: bool):
    """Q (B, H_q, 1, D); per_head (B, H_q, ...) the per-query-head selection
    (mask or id lists); call(Q_chunk, per_head_chunk) -> (O, lse).  Returns
    (O like Q, lse (B, H_q, 1) fp32 or None)."""
    H_q = Q.shape[1]
    nrep = H_q // H_kv
    O = torch.empty_like(Q)
    lse = torch.empty(Q.shape[0], H_q, 1, dtype=torch.float32, device=Q.device) if return_lse else None
    for off, size in head_chunks(nrep):
        oc, lc = call(heads(Q, 1, H_kv, nrep, off, size), heads(per_head, 1, H_kv, nrep, off, size))
        put_heads(O, oc, 1, H_kv, nrep, off, size)
        if lse is not None:
            put_heads(lse, lc, 1, H_kv, nrep, off, size)
    return O, lse

