"""The decode step of the reference's attention patch, on HIP.

Mirrors the S_q == 1 branch of make_quest_persistent_forward
(src/flashquest/eager/llama_persistent_patch.py:202-245): score the completed
pages from their K metadata, select pages, run sparse attention over the
packed cache, and merge with dense attention over the partial-page tail
(_bf16_dense_attn_with_lse 30-47, _merge_two_attentions 50-61).
"""
from __future__ import annotations

import math

import torch

from .. import _lib as L
from .. import _ops


def bf16_dense_attn_with_lse(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor):
    """llama_persistent_patch.py:30-47.  Q (B,H_q,1,D); K, V (B,H_kv,T,D).
    Returns (O (B,H_q,1,D) bf16, lse (B,H_q,1) fp32, natural log)."""
    L.require_device(Q, K, V)
    B, H_q, _, D = Q.shape
    H_kv, T = K.shape[1], K.shape[2]
    if K.dtype != V.dtype or Q.dtype != K.dtype:
        raise AssertionError("Q, K and V must share a dtype")
    Q3 = Q[:, :, 0, :]
    O = torch.empty(B, H_q, D, dtype=torch.bfloat16, device=Q.device)
    lse = torch.empty(B, H_q, dtype=torch.float32, device=Q.device)
    L.check(L.lib().fq_dense_tail_attn(Q3.data_ptr(), L.strides(Q3, 3), K.data_ptr(), L.strides(K, 4),
                                       V.data_ptr(), L.strides(V, 4), L.dtype_code(K.dtype), O.data_ptr(),
                                       L.strides(O, 3), lse.data_ptr(), B, H_q, H_kv, T, D,
                                       L.stream_handle(Q.device)), "bf16_dense_attn_with_lse")
    return O.unsqueeze(2), lse.unsqueeze(2)


def merge_two_attentions(O_a, lse_a, O_b, lse_b) -> torch.Tensor:
    """llama_persistent_patch.py:50-61: LSE-weighted merge, output in O_a's dtype."""
    L.require_device(O_a, O_b)
    D = O_a.shape[-1]
    oa = O_a.reshape(-1, D)
    ob = O_b.to(O_a.dtype).reshape(-1, D)
    la = lse_a.reshape(-1).float().contiguous()
    lb = lse_b.reshape(-1).float().contiguous()
    out = torch.empty_like(oa)
    N = oa.shape[0]
    L.check(L.lib().fq_merge_attn(oa.data_ptr(), la.data_ptr(), ob.data_ptr(), lb.data_ptr(),
                                  L.dtype_code(oa.dtype), oa.stride(0), ob.stride(0), out.data_ptr(),
                                  out.stride(0), None, N, D, L.stream_handle(O_a.device)),
            "merge_two_attentions")
    return out.view(O_a.shape)


_FUSED_TAIL_REFUSED = "the fused tail needs the matrix-core attention layout"


def _tail_by_merge(run_sparse, Q3, O3, lse, K_tail, V_tail, sm_scale):
    """The reference's own partial-page sequence (llama_persistent_patch.py:
    232-245) for the shapes whose fused tail the library refuses (GQA ratios
    above 4, head_dim 64, other page sizes): sparse attention over the
    completed pages into fp32 O and lse (run_sparse(O, lse)), then
    _bf16_dense_attn_with_lse over the tail (fp32 arithmetic, bf16 O, as
    there), then _merge_two_attentions (fp32, cast to O3's dtype)."""
    D = Q3.shape[-1]
    if sm_scale is not None and float(sm_scale) != 1.0 / math.sqrt(D):
        raise NotImplementedError("the partial-page merge takes the default sm_scale (1/sqrt(head_dim))")
    O_sp = torch.empty(Q3.shape, dtype=torch.float32, device=Q3.device)
    lse_sp = torch.empty(Q3.shape[:-1], dtype=torch.float32, device=Q3.device)
    run_sparse(O_sp, lse_sp)
    H_q, H_kv, T = Q3.shape[-2], K_tail.shape[-3], K_tail.shape[-2]
    n = O_sp.numel() // (H_q * D)
    q = Q3.reshape(n, H_q, 1, D).float()
    kt = K_tail.reshape(n, H_kv, T, D).float()
    vt = V_tail.reshape(n, H_kv, T, D).float()
    O_t, lse_t = bf16_dense_attn_with_lse(q, kt, vt)
    oa = O_sp.reshape(-1, D)
    ob = O_t.float().reshape(-1, D)
    la = lse_sp.reshape(-1).contiguous()
    lb = lse_t.reshape(-1).contiguous()
    merged = torch.empty_like(oa)
    lse_m = torch.empty_like(la)
    L.check(L.lib().fq_merge_attn(oa.data_ptr(), la.data_ptr(), ob.data_ptr(), lb.data_ptr(),
                                  L.dtype_code(oa.dtype), oa.stride(0), ob.stride(0), merged.data_ptr(),
                                  merged.stride(0), lse_m.data_ptr(), oa.shape[0], D, L.stream_handle(Q3.device)),
            "merge_two_attentions")
    O3.copy_(merged.view(O3.shape))
    if lse is not None:
        lse.copy_(lse_m.view(lse.shape))


def quest_decode_int4(
    Q: torch.Tensor,
    K_packed: torch.Tensor,
    K_scale: torch.Tensor,
    K_mn: torch.Tensor,
    V_packed: torch.Tensor,
    V_scale: torch.Tensor,
    V_mn: torch.Tensor,
    *,
    retention: float | torch.Tensor,
    num_sinks: int = 4,
    window_pages: int = 2,
    k_max_static: int | None = None,
    page_size: int = 64,
    select_mode: str = "per_q_head",
    sm_scale: float | None = None,
    return_lse: bool = True,
    return_selection: bool = False,
    out: torch.Tensor | None = None,
    K_tail: torch.Tensor | None = None,
    V_tail: torch.Tensor | None = None,
    head_pattern: torch.Tensor | None = None,
    rotation_signs: torch.Tensor | None = None,
    _rotation: torch.Tensor | None = None,
    _direct: bool = False,
):
    """Fused score -> select -> sparse attention over completed pages.

    One layer: Q (B,H_q,1,D), cache tensors 4D (B,H_kv,...).  L layers at once:
    Q (L,B,H_q,1,D), cache tensors 5D (L,B,H_kv,...), every layer independent.
    ``select_mode`` "per_q_head" is the reference's selection
    (selection.py:103-117); "per_kv_head_sum" selects once per KV head from
    the fp32 sum of its query heads' scores.
    ``K_tail`` / ``V_tail`` (..., H_kv, T, D), T <= 64: the partial page,
    attended with the selected pages (llama_persistent_patch.py:229-240); O and
    lse are then those of the merged attention.  Raises NotImplementedError for
    shapes the fused tail does not take (``sparse_decode_layer`` falls back).
    ``head_pattern`` (H_kv,) or (L, H_kv) bool: DuoAttention's per-KV-head
    retrieval (True) / streaming (False) pattern; streaming heads keep only
    the sink and window pages (llama_persistent_patch.py:214-220).
    ``rotation_signs`` (D,) +-1 (benchmark config 3, no reference function): the
    cache holds K and V rotated by x -> WHT(s x) / sqrt(D); Q is rotated the
    same way (fp32) before scoring and attention and O rotated back,
    O = s WHT(O_rot) / sqrt(D), lse unchanged (the rotation is orthogonal).
    The single-launch kernel does both in its prologue and epilogue; calls
    that take the split path rotate with fq_wht (fp32) around the step.
    Returns (O like Q, lse (..., H_q, 1) fp32 or None[, mask (..., H_q, P) bool]).
    """
    if select_mode not in L.SELECT_MODES:
        raise ValueError(f"select_mode must be one of {sorted(L.SELECT_MODES)}")
    L.require_device(Q, K_packed, K_scale)
    if Q.shape[-2] != 1:
        raise NotImplementedError(f"quest_decode_int4: decode-only (S_q={Q.shape[-2]})")
    if rotation_signs is not None:
        return _rotated_decode(Q, (K_packed, K_scale, K_mn, V_packed, V_scale, V_mn), rotation_signs, out,
                               dict(retention=retention, num_sinks=num_sinks, window_pages=window_pages,
                                    k_max_static=k_max_static, page_size=page_size, select_mode=select_mode,
                                    sm_scale=sm_scale, return_lse=return_lse, return_selection=return_selection,
                                    K_tail=K_tail, V_tail=V_tail, head_pattern=head_pattern))
    D = Q.shape[-1]
    if D not in (64, 128):
        raise NotImplementedError(f"head_dim={D} not in (64, 128)")
    H_kv = K_scale.shape[-3]
    nrep = Q.shape[-3] // H_kv if Q.shape[-3] % H_kv == 0 else 0
    if (not _direct and _ops.wants_head_chunks(Q.shape[-3], H_kv, D, page_size) and _rotation is None
            and not _one_launch(4, Q, (K_packed, K_scale, K_mn, V_packed, V_scale, V_mn), nrep, page_size,
                                select_mode, num_sinks, window_pages, k_max_static)):
        planes = (K_packed, K_scale, K_mn, V_packed, V_scale, V_mn)
        kw = dict(retention=retention, num_sinks=num_sinks, window_pages=window_pages, k_max_static=k_max_static,
                  page_size=page_size, select_mode=select_mode, sm_scale=sm_scale, return_lse=return_lse,
                  return_selection=return_selection, K_tail=K_tail, V_tail=V_tail, head_pattern=head_pattern)
        res = _padded_decode(4, Q, planes, H_kv, nrep, out, kw) if nrep in (5, 7) else None
        return res if res is not None else _chunked_decode(4, Q, planes, H_kv, nrep, out, kw)
    layered = Q.dim() == 5
    Q3 = Q[..., 0, :]
    H_q = Q3.shape[-2]
    P = K_scale.shape[-2]
    O3 = torch.empty_like(Q3) if out is None else out[..., 0, :]
    lse = torch.empty(Q3.shape[:-1], dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size)
    if H_q % cache.H_kv:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={cache.H_kv}")
    query = _ops.query(Q3, O3, lse, sm_scale)
    r, query.retention_layer_stride = _ops.retention_rows(retention, head_pattern, H_q, cache.H_kv,
                                                          Q3.shape[0] if Q3.dim() == 4 else 1, Q.device)
    query.rotation_signs = None if _rotation is None else _rotation.data_ptr()
    k_max = -1 if k_max_static is None else min(int(k_max_static), P)
    mask = None
    if return_selection:
        mask = torch.empty(Q3.shape[:-1] + (P,), dtype=torch.bool, device=Q.device)
    stream = L.stream_handle(Q.device)
    ws = L.workspace(Q.device, L.lib().fq_workspace_bytes(cache, H_q), stream)
    tail, tail_keep = _tail(K_tail, V_tail, D, return_selection)
    if tail is not None:
        try:
            L.check(L.lib().fq_quest_decode_int4_tail(cache, query, tail, r.data_ptr(), int(num_sinks),
                                                      int(window_pages), k_max, L.SELECT_MODES[select_mode],
                                                      ws.data_ptr(), ws.numel(), stream),
                    "quest_decode_int4 (tail)")
        except NotImplementedError as e:
            if _FUSED_TAIL_REFUSED not in str(e) or _rotation is not None:
                raise

            def run_sparse(O_sp, lse_sp):
                q2 = _ops.query(Q3, O_sp, lse_sp, sm_scale)
                q2.retention_layer_stride = query.retention_layer_stride
                L.check(L.lib().fq_quest_decode_int4(cache, q2, r.data_ptr(), int(num_sinks), int(window_pages),
                                                     k_max, L.SELECT_MODES[select_mode], None, None,
                                                     ws.data_ptr(), ws.numel(), stream), "quest_decode_int4")
            _tail_by_merge(run_sparse, Q3, O3, lse, tail_keep[0], tail_keep[1], sm_scale)
    else:
        L.check(L.lib().fq_quest_decode_int4(cache, query, r.data_ptr(), int(num_sinks), int(window_pages), k_max,
                                             L.SELECT_MODES[select_mode], None,
                                             None if mask is None else mask.data_ptr(),
                                             ws.data_ptr(), ws.numel(), stream),
                "quest_decode_int4")
    O = O3.unsqueeze(-2)
    lse_out = lse.unsqueeze(-1) if lse is not None else None
    if return_selection:
        return O, lse_out, mask
    return O, lse_out


def _one_launch(bits, Q, planes, nrep, page_size, select_mode, num_sinks, window_pages, k_max_static, raw=None):
    """True when fq_quest_decode_int4 / _int8 / _turbo (bits 4 / 8 / 3; raw:
    TurboQuant's (K_scale_raw, K_mn_raw)) takes a step of 6 or 8 query heads
    per KV head as one launch itself: with enough KV groups the library runs
    every KV head as two virtual heads of 3 or 4 query heads, one workgroup
    each."""
    if nrep not in (6, 8):
        return False
    Q3 = Q[..., 0, :]
    probe = _ops.query(Q3, Q3, None, None)
    if bits == 3:
        cache, keep = _ops.turbo_cache(*planes, raw[0].shape[-2], page_size)
        return L.lib().fq_quest_fused_turbo(cache, probe) == 1
    cache, keep = (_ops.int4_cache if bits == 4 else _ops.int8_cache)(*planes, page_size)
    P = planes[1].shape[-2]
    k_max = -1 if k_max_static is None else min(int(k_max_static), P)
    fused = L.lib().fq_quest_fused_int4 if bits == 4 else L.lib().fq_quest_fused_int8
    return fused(cache, probe, int(num_sinks), int(window_pages), k_max, L.SELECT_MODES[select_mode]) == 1


def _pad_heads(x, axis: int, H_kv: int, nrep: int, fill: float = 0.0):
    """x with one more head per KV group on its (group-major) head axis `axis`,
    the new last head of every group filled with `fill`."""
    g = x.unflatten(axis, (H_kv, nrep))
    shape = list(g.shape)
    shape[axis + 1] = 1
    return torch.cat([g, torch.full(shape, fill, dtype=x.dtype, device=x.device)], dim=axis + 1).flatten(axis, axis + 1)


def _real_heads(x, axis: int, H_kv: int, nrep: int, grouped: bool = False):
    """The nrep real heads of every group of a tensor padded by _pad_heads: a
    view with the heads as (H_kv, nrep) when `grouped` (writable in place),
    else flattened back to H_kv * nrep heads (a copy)."""
    g = x.unflatten(axis, (H_kv, nrep + 1)).narrow(axis + 1, 0, nrep)
    return g if grouped else g.flatten(axis, axis + 1)


_padded_scalar = {}


def _padded_retention(retention, H_q: int, H_kv: int, nrep: int, device):
    """The per-head retention of a padded step: the real heads' values, 0 for
    the extra head of every group (it then selects only the forced pages).
    Scalar retentions are kept per (value, shape, device) outside graph
    capture, like _ops.retention_tensor's vectors."""
    if torch.is_tensor(retention):
        return _pad_heads(_ops.retention_tensor(retention, H_q, device), 0, H_kv, nrep)
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (float(retention), H_q, H_kv, nrep, device.type, device.index)
    r = _padded_scalar.get(key)
    if r is None:
        r = _pad_heads(_ops.retention_tensor(retention, H_q, device), 0, H_kv, nrep)
        capturing = device.type == "cuda" and torch.cuda.is_current_stream_capturing()
        if not capturing and len(_padded_scalar) < 64:
            _padded_scalar[key] = r
    return r


def _padded_decode(bits, Q, planes, H_kv, nrep, out, kw, raw=None):
    """quest_decode_int4 / _int8 / _turbo (bits 4 / 8 / 3) for 5 or 7 query
    heads per KV head as one step of 6 or 8: a zero query head is added to
    every KV group, with retention 0, so the library runs each KV head as two
    virtual heads of 3 or 4 query heads.  The extra head changes nothing the
    real heads see: its selection is the forced pages, which every head holds
    already; a per_kv_head_sum row adds 0 to the summed query (exact in fp32)
    and its k comes from the largest retention, never 0's; its own output is
    dropped.  Returns None when the library would not take the padded step in
    its matrix-core kernels (the caller then attends in chunks)."""
    head_axis = Q.dim() - 3
    Qp = _pad_heads(Q, head_axis, H_kv, nrep)
    if not _one_launch(bits, Qp, planes, nrep + 1, kw["page_size"], kw["select_mode"], kw["num_sinks"],
                       kw["window_pages"], kw["k_max_static"], raw=raw):
        return None
    # _direct: the library takes the padded step (just checked), no second check
    sub = dict(kw, retention=_padded_retention(kw["retention"], Q.shape[-3], H_kv, nrep, Q.device), _direct=True)
    if bits == 3:
        res = quest_decode_turbo(Qp, *planes, *raw, **sub)
    else:
        res = (quest_decode_int4 if bits == 4 else quest_decode_int8)(Qp, *planes, **sub)
    O = _real_heads(res[0], head_axis, H_kv, nrep)
    if out is not None:
        out.copy_(O)
        O = out
    else:
        O = O.contiguous()
    lse = None if res[1] is None else _real_heads(res[1], res[1].dim() - 2, H_kv, nrep).contiguous()
    if kw["return_selection"]:
        return O, lse, _real_heads(res[2], res[2].dim() - 2, H_kv, nrep).contiguous()
    return O, lse


def _chunked_decode(bits, Q, planes, H_kv, nrep, out, kw, raw=None):
    """quest_decode_int4 / quest_decode_int8 / quest_decode_turbo (bits 4 / 8
    / 3; raw: TurboQuant's (K_scale_raw, K_mn_raw)) for more than 4 query
    heads per KV head (the reference's kernels take any ratio,
    sparse_int4_fwd.py:54-55, sparse_turbo_fwd.py): the group's query heads in
    chunks of at most 4, each on the matrix-core kernels where the layout
    allows (head_dim 128, 64-token pages).  per_q_head selects every head on
    its own, so each chunk is an ordinary step over its heads (any ratio).
    per_kv_head_sum selects once per KV group from all of its heads (one
    selection pass over the whole query, its mask kept; at most 8 heads, one
    mask bit each), then each chunk attends the group's pages through the
    mask entry.  A partial-page tail is merged as the reference does
    (llama_persistent_patch.py:232-245)."""
    head_axis = Q.dim() - 3
    # pages: K_scale (..., P, D) for INT4 / INT8; TurboQuant's planes are per
    # token, its page count is the raw K metadata's (..., P, D)
    H_q, D = Q.shape[-3], Q.shape[-1]
    P = raw[0].shape[-2] if bits == 3 else planes[1].shape[-2]
    O = torch.empty_like(Q) if out is None else out
    lse = torch.empty(Q.shape[:-2], dtype=torch.float32, device=Q.device) if kw["return_lse"] else None
    mask = torch.empty(Q.shape[:-2] + (P,), dtype=torch.bool, device=Q.device) if kw["return_selection"] else None
    retention = kw["retention"]

    def ret_chunk(off, size):
        if not torch.is_tensor(retention):
            return retention
        r = retention.to(device=Q.device, dtype=torch.float32)
        return _ops.heads(r, r.dim() - 1, H_kv, nrep, off, size)

    if kw["select_mode"] == "per_q_head":
        for off, size in _ops.head_chunks(nrep):
            sub = dict(kw, retention=ret_chunk(off, size))
            qc = _ops.heads(Q, head_axis, H_kv, nrep, off, size)
            if bits == 3:
                res = quest_decode_turbo(qc, *planes, *raw, **sub)
            else:
                res = (quest_decode_int4 if bits == 4 else quest_decode_int8)(qc, *planes, **sub)
            _ops.put_heads(O, res[0], head_axis, H_kv, nrep, off, size)
            if lse is not None:
                _ops.put_heads(lse, res[1][..., 0], head_axis, H_kv, nrep, off, size)
            if mask is not None:
                _ops.put_heads(mask, res[2], head_axis, H_kv, nrep, off, size)
        O_out = O
    else:
        if nrep > 8:
            raise NotImplementedError(f"per_kv_head_sum selects from one mask bit per query head of a KV group: "
                                      f"at most 8 query heads per KV head, got {nrep} (per_q_head takes any ratio)")
        if kw.get("K_tail") is not None and kw["K_tail"].shape[-2] > 0 and kw["return_selection"]:
            raise ValueError("return_selection is not available together with a fused tail")
        Q3 = Q[..., 0, :]
        lib = L.lib()
        if bits == 4:
            cache, keep = _ops.int4_cache(*planes, kw["page_size"])
            ws_bytes, select, attend = lib.fq_workspace_bytes, lib.fq_quest_select_int4, lib.fq_sparse_int4_fwd_mask
        elif bits == 8:
            cache, keep = _ops.int8_cache(*planes, kw["page_size"])
            ws_bytes, select, attend = (lib.fq_int8_workspace_bytes, lib.fq_quest_select_int8,
                                        lib.fq_sparse_int8_fwd_mask)
        else:
            cache, keep = _ops.turbo_cache(*planes, P, kw["page_size"])
            ksr, kmr = (x if x.stride(-1) == 1 else x.contiguous() for x in raw)
            lead = 5 - ksr.dim()

            def select(c, qd, *args):        # the raw K metadata goes before the query
                return lib.fq_quest_select_turbo(c, ksr.data_ptr(), L.strides(ksr, 5, lead), kmr.data_ptr(),
                                                 L.strides(kmr, 5, lead), qd, *args[:5], *args[6:])
            ws_bytes, attend = lib.fq_turbo_workspace_bytes, lib.fq_sparse_turbo_fwd_mask
        name = "quest_decode_turbo" if bits == 3 else f"quest_decode_int{bits}"
        stream = L.stream_handle(Q.device)
        sel = torch.empty(Q3.shape[:-1] + (P,), dtype=torch.uint8, device=Q.device)
        query = _ops.query(Q3, torch.empty_like(Q3), None, kw["sm_scale"])     # the selection writes no O
        r, query.retention_layer_stride = _ops.retention_rows(retention, kw["head_pattern"], H_q, H_kv,
                                                              Q3.shape[0] if Q3.dim() == 4 else 1, Q.device)
        k_max = -1 if kw["k_max_static"] is None else min(int(kw["k_max_static"]), P)
        ws = L.workspace(Q.device, ws_bytes(cache, H_q), stream)
        L.check(select(cache, query, r.data_ptr(), int(kw["num_sinks"]), int(kw["window_pages"]), k_max,
                       L.SELECT_MODES["per_kv_head_sum"], None, sel.data_ptr(), ws.data_ptr(), ws.numel(), stream),
                f"{name} (selection)")

        def run_sparse(O3, lse3):
            for off, size in _ops.head_chunks(nrep):
                qc = _ops.heads(Q3, Q3.dim() - 2, H_kv, nrep, off, size)
                mc = _ops.heads(sel, sel.dim() - 2, H_kv, nrep, off, size)
                oc = torch.empty(qc.shape, dtype=O3.dtype, device=Q.device)
                lc = torch.empty(qc.shape[:-1], dtype=torch.float32, device=Q.device)
                qd = _ops.query(qc, oc, lc, kw["sm_scale"])
                wsc = L.workspace(Q.device, ws_bytes(cache, qc.shape[-2]), stream)
                L.check(attend(cache, qd, mc.data_ptr(), L.strides(mc, 4, 4 - mc.dim()), wsc.data_ptr(), wsc.numel(),
                               stream), f"{name} (attention)")
                _ops.put_heads(O3, oc, O3.dim() - 2, H_kv, nrep, off, size)
                _ops.put_heads(lse3, lc, lse3.dim() - 1, H_kv, nrep, off, size)

        O3 = O[..., 0, :]
        lse3 = lse if lse is not None else torch.empty(Q3.shape[:-1], dtype=torch.float32, device=Q.device)
        if kw.get("K_tail") is not None and kw["K_tail"].shape[-2] > 0:
            _tail_by_merge(run_sparse, Q3, O3, lse3, kw["K_tail"], kw["V_tail"], kw["sm_scale"])
        else:
            run_sparse(O3, lse3)
        if mask is not None:
            mask.copy_(sel.bool())
        O_out = O
    lse_out = lse.unsqueeze(-1) if lse is not None else None
    if kw["return_selection"]:
        return O_out, lse_out, mask
    return O_out, lse_out


def _tail(K_tail, V_tail, D, return_selection):
    """The fused step's partial-page tail descriptor (None without a tail) and
    the tensors it points into."""
    if K_tail is None or K_tail.shape[-2] == 0:
        return None, ()
    if return_selection:
        raise ValueError("return_selection is not available together with a fused tail")
    L.require_device(K_tail, V_tail)
    if K_tail.shape != V_tail.shape or K_tail.dtype != V_tail.dtype or K_tail.shape[-1] != D:
        raise AssertionError("K_tail / V_tail must share shape (..., H_kv, T, D) and dtype")
    kt = K_tail if K_tail.stride(-1) == 1 else K_tail.contiguous()
    vt = V_tail if V_tail.stride(-1) == 1 else V_tail.contiguous()
    lead = 5 - kt.dim()
    tail = L.Tail(kt.data_ptr(), L.strides(kt, 5, lead), vt.data_ptr(), L.strides(vt, 5, lead),
                  L.dtype_code(kt.dtype), kt.shape[-2], D)
    return tail, (kt, vt)


def _signs(rotation_signs, D, device):
    s = rotation_signs.to(device=device, dtype=torch.float32).contiguous()
    if s.shape != (D,) or not bool(((s == 1) | (s == -1)).all()):
        raise ValueError(f"rotation_signs must be a ({D},) vector of +-1")
    return s


def _rotated_decode(Q, planes, rotation_signs, out, kw):
    """quest_decode_int4 with rotation_signs: the kernel's own rotation when
    the step is one launch, else fq_wht in fp32 around the split-path step."""
    from ..kernel.wht import wht_along_head_dim
    D = Q.shape[-1]
    if D != 128:
        raise NotImplementedError("the rotated decode takes head_dim 128")
    signs = _signs(rotation_signs, D, Q.device)
    Q3 = Q[..., 0, :]
    cache, keep = _ops.int4_cache(*planes, kw["page_size"])
    probe = _ops.query(Q3, Q3, None, None)
    k_max = -1 if kw["k_max_static"] is None else min(int(kw["k_max_static"]), planes[1].shape[-2])
    fused = L.lib().fq_quest_fused_int4(cache, probe, int(kw["num_sinks"]), int(kw["window_pages"]), k_max,
                                        L.SELECT_MODES[kw["select_mode"]]) == 1
    if fused:
        return quest_decode_int4(Q, *planes, out=out, _rotation=signs, **kw)
    q_rot = wht_along_head_dim(Q.float(), signs=signs)            # fp32 in, fp32 butterflies
    res = quest_decode_int4(q_rot, *planes, **kw)
    o = wht_along_head_dim(res[0], signs=signs, inverse=True).to(Q.dtype)
    if out is not None:
        out.copy_(o)
        o = out
    return (o,) + tuple(res[1:])


def quest_decode_int8(
    Q: torch.Tensor,
    K_uint8: torch.Tensor,
    K_scale: torch.Tensor,
    K_mn: torch.Tensor,
    V_uint8: torch.Tensor,
    V_scale: torch.Tensor,
    V_mn: torch.Tensor,
    *,
    retention: float | torch.Tensor,
    num_sinks: int = 4,
    window_pages: int = 2,
    k_max_static: int | None = None,
    page_size: int = 64,
    select_mode: str = "per_q_head",
    sm_scale: float | None = None,
    return_lse: bool = True,
    return_selection: bool = False,
    head_pattern: torch.Tensor | None = None,
    K_tail: torch.Tensor | None = None,
    V_tail: torch.Tensor | None = None,
    _direct: bool = False,
):
    """The INT8 decode step (llama_persistent_patch.py:143-160 with the
    selection of 196-245): page_scores_int8_fast -> select_pages_vectorized ->
    flash_attn_sparse_fwd over the completed pages, for one layer (Q
    (B,H_q,1,D), 4D cache) or L layers at once (Q (L,B,H_q,1,D), 5D cache).
    ``select_mode``, ``head_pattern`` and ``K_tail`` / ``V_tail`` (the
    partial page, attended and merged in the same step) as quest_decode_int4.
    Returns (O like Q, lse (..., H_q, 1) fp32 or None[, mask (..., H_q, P)
    bool])."""
    if select_mode not in L.SELECT_MODES:
        raise ValueError(f"select_mode must be one of {sorted(L.SELECT_MODES)}")
    L.require_device(Q, K_uint8, K_scale)
    if Q.shape[-2] != 1:
        raise NotImplementedError(f"quest_decode_int8: decode-only (S_q={Q.shape[-2]})")
    D = Q.shape[-1]
    if D not in (64, 128):
        raise NotImplementedError(f"head_dim={D} not in (64, 128)")
    H_kv = K_scale.shape[-3]
    nrep = Q.shape[-3] // H_kv if Q.shape[-3] % H_kv == 0 else 0
    if (not _direct and _ops.wants_head_chunks(Q.shape[-3], H_kv, D, page_size)
            and not _one_launch(8, Q, (K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn), nrep, page_size,
                                select_mode, num_sinks, window_pages, k_max_static)):
        planes = (K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn)
        kw = dict(retention=retention, num_sinks=num_sinks, window_pages=window_pages, k_max_static=k_max_static,
                  page_size=page_size, select_mode=select_mode, sm_scale=sm_scale, return_lse=return_lse,
                  return_selection=return_selection, K_tail=K_tail, V_tail=V_tail, head_pattern=head_pattern)
        res = _padded_decode(8, Q, planes, H_kv, nrep, None, kw) if nrep in (5, 7) else None
        return res if res is not None else _chunked_decode(8, Q, planes, H_kv, nrep, None, kw)
    Q3 = Q[..., 0, :]
    H_q = Q3.shape[-2]
    P = K_scale.shape[-2]
    O3 = torch.empty_like(Q3)
    lse = torch.empty(Q3.shape[:-1], dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.int8_cache(K_uint8, K_scale, K_mn, V_uint8, V_scale, V_mn, page_size)
    if H_q % cache.H_kv:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={cache.H_kv}")
    query = _ops.query(Q3, O3, lse, sm_scale)
    r, query.retention_layer_stride = _ops.retention_rows(retention, head_pattern, H_q, cache.H_kv,
                                                          Q3.shape[0] if Q3.dim() == 4 else 1, Q.device)
    k_max = -1 if k_max_static is None else min(int(k_max_static), P)
    mask = torch.empty(Q3.shape[:-1] + (P,), dtype=torch.bool, device=Q.device) if return_selection else None
    stream = L.stream_handle(Q.device)
    ws = L.workspace(Q.device, L.lib().fq_int8_workspace_bytes(cache, H_q), stream)
    tail, tail_keep = _tail(K_tail, V_tail, D, return_selection)
    if tail is not None:
        try:
            L.check(L.lib().fq_quest_decode_int8_tail(cache, query, tail, r.data_ptr(), int(num_sinks),
                                                      int(window_pages), k_max, L.SELECT_MODES[select_mode],
                                                      ws.data_ptr(), ws.numel(), stream),
                    "quest_decode_int8 (tail)")
        except NotImplementedError as e:
            if _FUSED_TAIL_REFUSED not in str(e):
                raise

            def run_sparse(O_sp, lse_sp):
                q2 = _ops.query(Q3, O_sp, lse_sp, sm_scale)
                q2.retention_layer_stride = query.retention_layer_stride
                L.check(L.lib().fq_quest_decode_int8(cache, q2, r.data_ptr(), int(num_sinks), int(window_pages),
                                                     k_max, L.SELECT_MODES[select_mode], None, None,
                                                     ws.data_ptr(), ws.numel(), stream), "quest_decode_int8")
            _tail_by_merge(run_sparse, Q3, O3, lse, tail_keep[0], tail_keep[1], sm_scale)
    else:
        L.check(L.lib().fq_quest_decode_int8(cache, query, r.data_ptr(), int(num_sinks), int(window_pages), k_max,
                                             L.SELECT_MODES[select_mode], None,
                                             None if mask is None else mask.data_ptr(),
                                             ws.data_ptr(), ws.numel(), stream),
                "quest_decode_int8")
    O = O3.unsqueeze(-2)
    lse_out = lse.unsqueeze(-1) if lse is not None else None
    if return_selection:
        return O, lse_out, mask
    return O, lse_out


def quest_decode_turbo(
    Q: torch.Tensor,
    K_msb: torch.Tensor,
    K_lsb: torch.Tensor,
    K_scale_turbo: torch.Tensor,
    V_msb: torch.Tensor,
    V_lsb: torch.Tensor,
    V_scale_turbo: torch.Tensor,
    K_scale_raw: torch.Tensor,
    K_mn_raw: torch.Tensor,
    *,
    retention: float | torch.Tensor,
    num_sinks: int = 4,
    window_pages: int = 2,
    k_max_static: int | None = None,
    page_size: int = 64,
    select_mode: str = "per_q_head",
    sm_scale: float | None = None,
    return_lse: bool = True,
    return_selection: bool = False,
    head_pattern: torch.Tensor | None = None,
    _direct: bool = False,
):
    """The reference's TurboQuant decode over completed pages, fused: page scores
    from the un-rotated K page metadata (criticality.py:128-163), selection
    (selection.py:65-126), flash_attn_sparse_turbo_fwd (sparse_turbo_fwd.py:254-346).

    One layer: Q (B,H_q,1,D) raw basis, cache tensors 4D (B,H_kv,...).  L layers
    at once: Q (L,B,H_q,1,D), cache tensors 5D.  ``head_pattern`` as
    quest_decode_int4.  Returns (O like Q in the raw basis, lse (..., H_q, 1)
    fp32 or None[, mask (..., H_q, P) bool]).
    """
    if select_mode not in L.SELECT_MODES:
        raise ValueError(f"select_mode must be one of {sorted(L.SELECT_MODES)}")
    L.require_device(Q, K_msb, K_scale_raw)
    if Q.shape[-2] != 1:
        raise NotImplementedError(f"quest_decode_turbo: decode-only (S_q={Q.shape[-2]})")
    D = Q.shape[-1]
    if D not in (64, 128):
        raise NotImplementedError(f"head_dim={D} not in (64, 128)")
    if K_scale_raw.dtype != torch.bfloat16 or K_mn_raw.dtype != torch.bfloat16:
        raise AssertionError("K_scale_raw / K_mn_raw must be bf16")
    H_kv = K_msb.shape[-3]
    nrep = Q.shape[-3] // H_kv if Q.shape[-3] % H_kv == 0 else 0
    if (not _direct and _ops.wants_head_chunks(Q.shape[-3], H_kv, D, page_size)
            and not _one_launch(3, Q, (K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo), nrep, page_size,
                                select_mode, num_sinks, window_pages, k_max_static, raw=(K_scale_raw, K_mn_raw))):
        planes = (K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo)
        kw = dict(retention=retention, num_sinks=num_sinks, window_pages=window_pages, k_max_static=k_max_static,
                  page_size=page_size, select_mode=select_mode, sm_scale=sm_scale, return_lse=return_lse,
                  return_selection=return_selection, head_pattern=head_pattern)
        raw = (K_scale_raw, K_mn_raw)
        res = _padded_decode(3, Q, planes, H_kv, nrep, None, kw, raw=raw) if nrep in (5, 7) else None
        return res if res is not None else _chunked_decode(3, Q, planes, H_kv, nrep, None, kw, raw=raw)
    Q3 = Q[..., 0, :]
    H_q = Q3.shape[-2]
    P = K_scale_raw.shape[-2]
    O3 = torch.empty_like(Q3)
    lse = torch.empty(Q3.shape[:-1], dtype=torch.float32, device=Q.device) if return_lse else None
    cache, keep = _ops.turbo_cache(K_msb, K_lsb, K_scale_turbo, V_msb, V_lsb, V_scale_turbo, P, page_size)
    if H_q % cache.H_kv:
        raise ValueError(f"H_q={H_q} must be divisible by H_kv={cache.H_kv}")
    lead = 5 - K_scale_raw.dim()
    ksr = K_scale_raw if K_scale_raw.stride(-1) == 1 else K_scale_raw.contiguous()
    kmr = K_mn_raw if K_mn_raw.stride(-1) == 1 else K_mn_raw.contiguous()
    query = _ops.query(Q3, O3, lse, sm_scale)
    r, query.retention_layer_stride = _ops.retention_rows(retention, head_pattern, H_q, cache.H_kv,
                                                          Q3.shape[0] if Q3.dim() == 4 else 1, Q.device)
    k_max = -1 if k_max_static is None else min(int(k_max_static), P)
    mask = None
    if return_selection:
        mask = torch.empty(Q3.shape[:-1] + (P,), dtype=torch.bool, device=Q.device)
    stream = L.stream_handle(Q.device)
    ws = L.workspace(Q.device, L.lib().fq_turbo_workspace_bytes(cache, H_q), stream)
    L.check(L.lib().fq_quest_decode_turbo(cache, ksr.data_ptr(), L.strides(ksr, 5, lead), kmr.data_ptr(),
                                          L.strides(kmr, 5, lead), query, r.data_ptr(), int(num_sinks),
                                          int(window_pages), k_max, L.SELECT_MODES[select_mode],
                                          None if mask is None else mask.data_ptr(), ws.data_ptr(), ws.numel(),
                                          stream), "quest_decode_turbo")
    O = O3.unsqueeze(-2)
    lse_out = lse.unsqueeze(-1) if lse is not None else None
    if return_selection:
        return O, lse_out, mask
    return O, lse_out


class QuestDecoder:
    """A reusable fused decode over fixed cache tensors (the bench's timed unit).

    Builds the C descriptors once; ``select()`` (scoring, and the selection
    kernel where the attention kernel does not select for itself) and
    ``attend()`` are the two halves of fq_quest_decode_int4, ``__call__`` runs
    both.
    Every launch goes to torch's current stream, so the calls can be captured
    in a HIP graph after one eager call has sized the workspace.  With more
    than 4 query heads per KV head the step is quest_decode_int4's chunked
    one, unless the library takes it as one launch (6 or 8 query heads per KV
    head, enough KV groups to fill the GPU).
    """

    def __init__(self, Q, K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, *, retention, num_sinks=4,
                 window_pages=2, k_max_static=None, page_size=64, select_mode="per_q_head", sm_scale=None,
                 out=None, lse=None, mask_out=None, K_tail=None, V_tail=None, head_pattern=None,
                 rotation_signs=None):
        if select_mode not in L.SELECT_MODES:
            raise ValueError(f"select_mode must be one of {sorted(L.SELECT_MODES)}")
        self.Q3 = Q[..., 0, :]
        self.O3 = torch.empty_like(self.Q3) if out is None else out[..., 0, :]
        self.lse = lse
        self.device = Q.device
        self.tail = None
        # more than 4 query heads per KV head, not one launch in the library:
        # the step is quest_decode_int4's chunked one (its tensors come from
        # the graph's pool when captured; the retention is moved to the device
        # here, not during a capture)
        self._chunked = None
        self._padded = None
        H_kv = K_scale.shape[-3]
        nrep = Q.shape[-3] // H_kv if Q.shape[-3] % H_kv == 0 else 0
        planes = (K_packed, K_scale, K_mn, V_packed, V_scale, V_mn)
        wants = (_ops.wants_head_chunks(Q.shape[-3], H_kv, Q.shape[-1], page_size)
                 and rotation_signs is None and mask_out is None
                 and not _one_launch(4, Q, planes, nrep, page_size, select_mode, num_sinks, window_pages,
                                     k_max_static))
        if wants and nrep in (5, 7):
            # 5 or 7 query heads per KV head: a step of 6 or 8 with a zero query
            # head per group (quest_decode_int4's padded step) when the library
            # takes that in its matrix-core kernels; q is copied in and O out
            axis = Q.dim() - 3
            Qp = _pad_heads(Q, axis, H_kv, nrep)
            if _one_launch(4, Qp, planes, nrep + 1, page_size, select_mode, num_sinks, window_pages, k_max_static):
                self._Op = torch.empty_like(Qp)
                self._lsep = None if lse is None else torch.empty(Qp.shape[:-2], dtype=torch.float32,
                                                                  device=Q.device)
                rp = _padded_retention(retention, Q.shape[-3], H_kv, nrep, Q.device)
                self._inner = QuestDecoder(Qp, *planes, retention=rp, num_sinks=num_sinks,
                                           window_pages=window_pages, k_max_static=k_max_static,
                                           page_size=page_size, select_mode=select_mode, sm_scale=sm_scale,
                                           out=self._Op, lse=self._lsep, K_tail=K_tail, V_tail=V_tail,
                                           head_pattern=head_pattern)
                # in-place views: the real heads of the padded query and output
                # beside the caller's, both as (H_kv, nrep)
                self._padded = (Q.unflatten(axis, (H_kv, nrep)), _real_heads(Qp, axis, H_kv, nrep, grouped=True),
                                _real_heads(self._Op[..., 0, :], axis, H_kv, nrep, grouped=True),
                                self.O3.unflatten(axis, (H_kv, nrep)),
                                None if lse is None else _real_heads(self._lsep, axis, H_kv, nrep, grouped=True),
                                None if lse is None else lse.unflatten(axis, (H_kv, nrep)))
                return
        if wants:
            ret = retention.to(device=Q.device, dtype=torch.float32) if torch.is_tensor(retention) else retention
            self._chunked = (Q, planes,
                             dict(retention=ret, num_sinks=num_sinks, window_pages=window_pages,
                                  k_max_static=k_max_static, page_size=page_size, select_mode=select_mode,
                                  sm_scale=sm_scale, return_lse=lse is not None, K_tail=K_tail, V_tail=V_tail,
                                  head_pattern=head_pattern))
            return
        self.cache, self._keep = _ops.int4_cache(K_packed, K_scale, K_mn, V_packed, V_scale, V_mn, page_size)
        self.query = _ops.query(self.Q3, self.O3, lse, sm_scale)
        H_q = self.Q3.shape[-2]
        P = K_scale.shape[-2]
        self._signs = None if rotation_signs is None else _signs(rotation_signs, self.Q3.shape[-1], Q.device)
        self.query.rotation_signs = None if self._signs is None else self._signs.data_ptr()
        self.r, self.query.retention_layer_stride = _ops.retention_rows(
            retention, head_pattern, H_q, self.cache.H_kv, self.Q3.shape[0] if self.Q3.dim() == 4 else 1, Q.device)
        self.k_max = -1 if k_max_static is None else min(int(k_max_static), P)
        self.sinks, self.window = int(num_sinks), int(window_pages)
        self.mode = L.SELECT_MODES[select_mode]
        self.mask_out = mask_out
        self.device = Q.device
        self.ws = L.workspace(Q.device, L.lib().fq_workspace_bytes(self.cache, H_q))
        self.tail = None
        if K_tail is not None and K_tail.shape[-2] > 0:
            lead = 5 - K_tail.dim()
            self._tail_keep = (K_tail, V_tail)
            self.tail = L.Tail(K_tail.data_ptr(), L.strides(K_tail, 5, lead), V_tail.data_ptr(),
                               L.strides(V_tail, 5, lead), L.dtype_code(K_tail.dtype), K_tail.shape[-2],
                               K_tail.shape[-1])

    @property
    def fused(self) -> bool:
        """True when attend() is the whole step: one attention kernel that scores
        and selects its own pages (select() then launches nothing)."""
        if self._padded is not None:
            return self._inner.fused
        if self._chunked is not None:
            return False
        r = L.lib().fq_quest_fused_int4(self.cache, self.query, self.sinks, self.window, self.k_max, self.mode)
        if r < 0:
            L.check(-r, "quest fused query")
        return r == 1

    def select(self):
        if self._padded is not None:       # q into the padded query, then its selection
            q_src, q_dst = self._padded[0], self._padded[1]
            q_dst.copy_(q_src)
            if self._inner.tail is None:
                self._inner.select()
            return
        if self._chunked is not None:      # the chunked step selects inside attend()
            return
        L.check(L.lib().fq_quest_select_int4(self.cache, self.query, self.r.data_ptr(), self.sinks, self.window,
                                             self.k_max, self.mode, None, L.ptr(self.mask_out), self.ws.data_ptr(),
                                             self.ws.numel(), L.stream_handle(self.device)), "quest select")

    def attend(self):
        if self._padded is not None:       # the padded step, then the real heads' O (and lse) out
            _, _, o_src, o_dst, l_src, l_dst = self._padded
            self._inner.attend()
            o_dst.copy_(o_src)
            if l_dst is not None:
                l_dst.copy_(l_src)
            return
        if self._chunked is not None:
            Q, planes, kw = self._chunked
            _, lse = quest_decode_int4(Q, *planes, out=self.O3.unsqueeze(-2), **kw)
            if self.lse is not None:
                self.lse.copy_(lse[..., 0])
            return
        if self.tail is not None:      # selection (when a kernel does it), attention, tail and merge
            L.check(L.lib().fq_quest_decode_int4_tail(self.cache, self.query, self.tail, self.r.data_ptr(),
                                                      self.sinks, self.window, self.k_max, self.mode,
                                                      self.ws.data_ptr(), self.ws.numel(),
                                                      L.stream_handle(self.device)), "quest attend (tail)")
            return
        L.check(L.lib().fq_quest_attend_int4(self.cache, self.query, self.r.data_ptr(), self.sinks, self.window,
                                             self.k_max, self.mode, self.ws.data_ptr(), self.ws.numel(),
                                             L.stream_handle(self.device)), "quest attend")

    def __call__(self):
        if self._padded is not None or (self._chunked is None and self.tail is None):
            self.select()
        self.attend()
        return self.O3.unsqueeze(-2)


def sparse_decode_layer(q: torch.Tensor, views: dict, *, retention, num_sinks: int, window_pages: int,
                        page_size: int, k_max_static: int | None = None, select_mode: str = "per_q_head",
                        head_pattern: torch.Tensor | None = None):
    """The decode branch of llama_persistent_patch.py:202-245 for one layer.

    ``views`` is get_views(layer) of a persistent INT4, INT8 or TurboQuant
    cache (persistent_int4.py:134-159, persistent_int8.py:137-169,
    persistent_turbo.py:149-176); the family follows from its keys, as the
    reference's kv_bits dispatch (llama_persistent_patch.py:74-163).
    ``head_pattern`` (H_kv,) bool: the layer's DuoAttention pattern
    (head_pattern_layer, llama_persistent_patch.py:214-220).
    Returns attention output (B, H_q, 1, D) in q's dtype.
    """
    completed = views["completed_len"]
    partial = views["partial_len"]
    if completed == 0:
        o, _ = bf16_dense_attn_with_lse(q, views["K_partial"], views["V_partial"])
        return o.to(q.dtype)
    kw = dict(retention=retention, num_sinks=num_sinks, window_pages=window_pages, k_max_static=k_max_static,
              page_size=page_size, select_mode=select_mode, head_pattern=head_pattern)
    if "K_uint8" in views:                    # INT8 (kv_bits 8)
        args = (q, views["K_uint8"], views["K_scale"], views["K_mn"], views["V_uint8"], views["V_scale"],
                views["V_mn"])
        if partial > 0:
            try:
                o, _ = quest_decode_int8(*args, K_tail=views["K_partial"], V_tail=views["V_partial"], **kw)
                return o
            except NotImplementedError:
                pass                          # layouts the fused tail does not take: three operators
        o_sparse, lse_sparse = quest_decode_int8(*args, **kw)
    elif "K_msb" in views:                    # TurboQuant K3-V3 (kv_bits 3)
        o_sparse, lse_sparse = quest_decode_turbo(q, views["K_msb"], views["K_lsb"], views["K_scale_turbo"],
                                                  views["V_msb"], views["V_lsb"], views["V_scale_turbo"],
                                                  views["K_scale_raw"], views["K_mn_raw"], **kw)
    else:                                     # INT4 (kv_bits 4)
        args = (q, views["K_packed"], views["K_scale"], views["K_mn"], views["V_packed"], views["V_scale"],
                views["V_mn"])
        if partial > 0:
            try:
                # one fused call: the tail is attended with the selected pages
                o, _ = quest_decode_int4(*args, K_tail=views["K_partial"], V_tail=views["V_partial"], **kw)
                return o
            except NotImplementedError:
                pass                          # layouts the fused tail does not take: three operators
        o_sparse, lse_sparse = quest_decode_int4(*args, **kw)
    if partial == 0:
        return o_sparse
    o_tail, lse_tail = bf16_dense_attn_with_lse(q.to(views["K_partial"].dtype), views["K_partial"],
                                                views["V_partial"])
    return merge_two_attentions(o_sparse, lse_sparse, o_tail, lse_tail)


def static_bucket(retention_max: float, max_seq_len: int, page_size: int, num_sinks: int, window_pages: int):
    """llama_persistent_patch.py:81-85: (k_max_static, bucket_max_static)."""
    k = math.ceil(retention_max * (max_seq_len // page_size))
    return k, k + num_sinks + window_pages
