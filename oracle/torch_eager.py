"""Eager PyTorch restatement of the reference's CPU-capable decode path, used
only as bench.py's CPU baseline (never by the product path).

TEST INFRASTRUCTURE ONLY.  The steps follow the reference's eager modules:
  1. page scores as two fp32 matmuls over the K metadata
     (src/flashquest/eager/criticality.py:128-163):
       s = q @ mn^T + 15 * relu(q) @ scale^T, per KV group of query heads;
  2. top-k per head plus the forced sink / window pages
     (src/flashquest/eager/selection.py:65-126), k = ceil(fp32(r) * fp32(P)),
     or once per KV head from the summed group scores ("per_kv_head_sum");
  3. fp32 dequantisation of the selected INT4 pages only
     (k = code * scale + mn; src/flashquest/kernel/sparse_int4_fwd.py:86-107);
  4. fp32 softmax attention over the selected tokens
     (scripts/profile_contribution.py:130-143).
"""
from __future__ import annotations

import math

import torch


def _unpack(packed: torch.Tensor) -> torch.Tensor:
    """(…, D/2) uint8 -> (…, D) fp32 codes, byte = c[2k] | c[2k+1] << 4."""
    lo = (packed & 0xF).to(torch.float32)
    hi = (packed >> 4).to(torch.float32)
    return torch.stack((lo, hi), dim=-1).flatten(-2)


def decode_layer(q, kp, ks, km, vp, vs, vm, *, retention: float, num_sinks: int = 4, window_pages: int = 2,
                 page: int = 64, select: str = "per_kv_head_sum", return_selection: bool = False):
    """One layer, batch 1.  q (H_q, D) fp32; kp/vp (H_kv, S, D/2) uint8;
    ks/km (H_kv, P, D); vs/vm (H_kv, S, G).  Returns O (H_q, D) fp32, and with
    return_selection also the page selection (H_q, P) bool."""
    Hq, D = q.shape
    Hkv, P = ks.shape[0], ks.shape[1]
    rep = Hq // Hkv
    qg = q.view(Hkv, rep, D)
    ksf, kmf = ks.float(), km.float()
    scores = torch.bmm(qg, kmf.transpose(1, 2)) + 15.0 * torch.bmm(qg.clamp_min(0), ksf.transpose(1, 2))
    k = min(P, math.ceil(float(torch.tensor(retention, dtype=torch.float32) * torch.tensor(float(P)))))
    forced = torch.zeros(P, dtype=torch.bool)
    forced[:min(num_sinks, P)] = True
    if window_pages > 0:
        forced[max(P - window_pages, 0):] = True
    if select == "per_kv_head_sum":
        top = scores.sum(1).topk(k, dim=-1).indices                         # (H_kv, k)
        sel = torch.zeros(Hkv, P, dtype=torch.bool)
        sel.scatter_(1, top, True)
        sel = (sel | forced).unsqueeze(1).expand(Hkv, rep, P)
    else:
        top = scores.topk(k, dim=-1).indices
        sel = torch.zeros(Hkv, rep, P, dtype=torch.bool)
        sel.scatter_(2, top, True)
        sel = sel | forced
    G = vs.shape[-1]
    out = torch.empty(Hkv, rep, D)
    scale = 1.0 / math.sqrt(D)
    for h in range(Hkv):
        pages = sel[h].any(0).nonzero().flatten()
        tok = (pages[:, None] * page + torch.arange(page)).flatten()
        kd = _unpack(kp[h, tok]) * ksf[h, pages].repeat_interleave(page, 0) + kmf[h, pages].repeat_interleave(page, 0)
        vd = _unpack(vp[h, tok]).view(-1, G, D // G) * vs[h, tok].float()[..., None] + vm[h, tok].float()[..., None]
        vd = vd.view(-1, D)
        logits = (qg[h] @ kd.T) * scale                                       # (rep, T)
        tok_mask = sel[h][:, pages].repeat_interleave(page, 1)
        logits = logits.masked_fill(~tok_mask, float("-inf"))
        out[h] = torch.softmax(logits, dim=-1) @ vd
    if return_selection:
        return out.view(Hq, D), sel.reshape(Hq, P)
    return out.view(Hq, D)
