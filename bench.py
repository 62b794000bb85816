"""Benchmark of the sparse INT4 decode-attention step on one MI355X.

Workload (benchmark config 1): 28 independent layers' KV caches, batch 1,
24 query / 8 KV heads, head_dim 128, 32k context = 512 pages of 64 tokens,
retention 0.25 (top-128 pages per KV head, per-KV-head selection from the
summed group scores) plus 4 sink and 2 window pages.  K/V are seeded synthetic
fp16 data (lognormal outlier channels in K, 4 planted pages per KV head),
quantised by this library to packed INT4 with fp16 metadata, V in 32-channel
groups.  One step = score + select + sparse attention for all 28 layers, with
L2 and the 256 MB MALL flushed before every step (outside the timed region).

Prints one JSON line (the driver's contract).  `--gpus N` with N > 1 exits:
this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from flashquest_amd._lib import KernelTimer  # noqa: E402
from flashquest_amd._probe import read_decode_pages, read_stream  # noqa: E402
from flashquest_amd.eager.decode import QuestDecoder  # noqa: E402
from flashquest_amd.kernel.kv_quant import (quantize_k, quantize_k_int4, quantize_k_turbo, quantize_v,  # noqa: E402
                                            quantize_v_int4, quantize_v_turbo)
from flashquest_amd.kernel.wht import wht_along_head_dim  # noqa: E402  (rotated caches, config 3)

METRIC = "decode-attn µs/step (28 layers, 32k, sparse INT4) + achieved HBM GB/s"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 matrix peak (no sparsity)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--pages", type=int, default=512)
    ap.add_argument("--retention", type=float, default=0.25)
    ap.add_argument("--select", default="per_kv_head_sum", choices=["per_kv_head_sum", "per_q_head"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip control / per-layer / per-q-head lines")
    ap.add_argument("--cpu-layers", type=int, default=10, help="layers in the CPU baseline sample")
    ap.add_argument("--no-batch16", dest="batch16", action="store_false",
                    help="skip the batch-16 line (benchmark config 4) among the extras")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="for rocprofv3 --pmc runs: a 256 MiB device copy (calibration), then 3 flushed steps")
    ap.add_argument("--profile-int8", action="store_true",
                    help="for rocprofv3 runs: 10 flushed fused INT8 decode steps (--select mode) only")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="for rocprofv3 runs: 8 prefills of a 32k-token prompt over one INT4 layer only "
                         "(3 to bring the clock up, then the 5 that are reported)")
    ap.add_argument("--profile-per-layer", action="store_true",
                    help="for rocprofv3 runs: the reference's per-layer call pattern (28 single-layer steps "
                         "in one HIP graph), 5 flushed replays only")
    ap.add_argument("--profile-turbo", action="store_true",
                    help="for rocprofv3 runs: 10 flushed fused TurboQuant decode steps (--select mode) only")
    ap.add_argument("--profile-gqa8", action="store_true",
                    help="for rocprofv3 runs: config 1 with 64 query heads (8 per KV head, two virtual KV heads "
                         "per KV head): a 256 MiB device copy (calibration), then 5 flushed steps (--select mode)")
    return ap.parse_args()


# --------------------------------------------------------------------- data --
ROT_SEED = 4242


def rotation_signs(D=128, dev="cuda"):
    """The seeded +-1 vector of the randomised WHT (benchmark config 3)."""
    g = torch.Generator()
    g.manual_seed(ROT_SEED)
    return (torch.randint(0, 2, (D,), generator=g) * 2 - 1).float().to(dev)


def gen_layer(l, b, Hq=24, Hkv=8, P=512, D=128, page=64, planted=4, dev="cuda"):
    """Seeded fp32 K, V (1, Hkv, S, D) and q (Hq, D) of (sequence b, layer l),
    seed 1000*b + l: N(0,1) K with lognormal(0,1) channel factors, 4 planted
    pages per KV head whose keys point along the group's mean query, N(0,1) V."""
    S = P * page
    rep = Hq // Hkv
    g = torch.Generator(device=dev)
    g.manual_seed(1000 * b + l)
    K = torch.randn(1, Hkv, S, D, generator=g, device=dev)
    K *= torch.exp(torch.randn(1, Hkv, 1, D, generator=g, device=dev))      # lognormal(0,1) channels
    V = torch.randn(1, Hkv, S, D, generator=g, device=dev)
    q = torch.randn(Hq, D, generator=g, device=dev)
    qhat = q.view(Hkv, rep, D).mean(1)
    qhat = qhat / qhat.norm(dim=-1, keepdim=True)
    rms = K[0].pow(2).mean(dim=(1, 2)).sqrt()
    for h in range(Hkv):
        pages = torch.randperm(P - 6, generator=g, device=dev)[:planted] + 4
        for p in pages.tolist():
            noise = torch.randn(page, D, generator=g, device=dev)
            K[0, h, p * page:(p + 1) * page] = rms[h] * (0.8 * math.sqrt(D) * qhat[h] + 0.6 * noise)
    return K, V, q


def make_cache(L, B, Hq=24, Hkv=8, P=512, D=128, page=64, planted=4, dev="cuda", signs=None):
    """Seeded synthetic INT4 cache, one (sequence, layer) at a time (gen_layer).
    With ``signs`` (config 3) K and V are rotated by WHT(signs * x) before
    quantisation; Q stays in the raw basis (the step rotates it)."""
    S = P * page
    kp = torch.empty(L, B, Hkv, S, D // 2, dtype=torch.uint8, device=dev)
    vp = torch.empty_like(kp)
    ks = torch.empty(L, B, Hkv, P, D, dtype=torch.float16, device=dev)
    km = torch.empty_like(ks)
    vs = torch.empty(L, B, Hkv, S, D // 32, dtype=torch.float16, device=dev)
    vm = torch.empty_like(vs)
    Q = torch.empty(L, B, Hq, 1, D, dtype=torch.float16, device=dev)
    for l in range(L):
        for b in range(B):
            K, V, q = gen_layer(l, b, Hq, Hkv, P, D, page, planted, dev)
            if signs is not None:
                K = wht_along_head_dim(K, signs=signs)
                V = wht_along_head_dim(V, signs=signs)
            quantize_k_int4(K.half(), page, out=(kp[l, b:b + 1], ks[l, b:b + 1], km[l, b:b + 1]))
            quantize_v_int4(V.half(), v_group=32, out=(vp[l, b:b + 1], vs[l, b:b + 1], vm[l, b:b + 1]))
            Q[l, b, :, 0] = q.half()
    torch.cuda.synchronize()
    return dict(Q=Q, K_packed=kp, K_scale=ks, K_mn=km, V_packed=vp, V_scale=vs, V_mn=vm)


def make_int8_cache(L, Hq=24, Hkv=8, P=512, D=128, page=64, dev="cuda"):
    """The same synthetic layers (batch 1) in the reference's INT8 layout
    (persistent_int8.py: uint8 codes, bf16 K page / V token metadata), layers
    folded into the batch axis, bf16 Q."""
    S = P * page
    c = {"K_uint8": torch.empty(L, Hkv, S, D, dtype=torch.uint8, device=dev),
         "K_scale": torch.empty(L, Hkv, P, D, dtype=torch.bfloat16, device=dev),
         "K_mn": torch.empty(L, Hkv, P, D, dtype=torch.bfloat16, device=dev),
         "V_uint8": torch.empty(L, Hkv, S, D, dtype=torch.uint8, device=dev),
         "V_scale": torch.empty(L, Hkv, S, 1, dtype=torch.bfloat16, device=dev),
         "V_mn": torch.empty(L, Hkv, S, 1, dtype=torch.bfloat16, device=dev),
         "Q": torch.empty(L, Hq, 1, D, dtype=torch.bfloat16, device=dev)}
    for l in range(L):
        K, V, q = gen_layer(l, 0, Hq, Hkv, P, D, page, 4, dev)
        quantize_k(K.bfloat16(), page, out=tuple(c[k][l:l + 1] for k in ("K_uint8", "K_scale", "K_mn")))
        quantize_v(V.bfloat16(), out=tuple(c[k][l:l + 1] for k in ("V_uint8", "V_scale", "V_mn")))
        c["Q"][l, :, 0] = q.bfloat16()
    torch.cuda.synchronize()
    return c


def make_turbo_cache(L, Hq=24, Hkv=8, P=512, D=128, page=64, dev="cuda"):
    """The same synthetic layers (batch 1) in the reference's TurboQuant K3-V3
    layout, layers folded into the batch axis: planes, per-token bf16 scales,
    the un-rotated K's bf16 page scale/min for scoring, bf16 Q."""
    S = P * page
    c = {"K_msb": torch.empty(L, Hkv, S, D // 8, dtype=torch.uint8, device=dev),
         "K_lsb": torch.empty(L, Hkv, S, D // 4, dtype=torch.uint8, device=dev),
         "K_scale_turbo": torch.empty(L, Hkv, S, 1, dtype=torch.bfloat16, device=dev),
         "K_scale_raw": torch.empty(L, Hkv, P, D, dtype=torch.bfloat16, device=dev),
         "K_mn_raw": torch.empty(L, Hkv, P, D, dtype=torch.bfloat16, device=dev),
         "V_msb": torch.empty(L, Hkv, S, D // 8, dtype=torch.uint8, device=dev),
         "V_lsb": torch.empty(L, Hkv, S, D // 4, dtype=torch.uint8, device=dev),
         "V_scale_turbo": torch.empty(L, Hkv, S, 1, dtype=torch.bfloat16, device=dev),
         "Q": torch.empty(L, Hq, 1, D, dtype=torch.bfloat16, device=dev)}
    for l in range(L):
        K, V, q = gen_layer(l, 0, Hq, Hkv, P, D, page, 4, dev)
        quantize_k_turbo(K.bfloat16(), page, out=tuple(c[k][l:l + 1] for k in
                                                       ("K_msb", "K_lsb", "K_scale_turbo", "K_scale_raw", "K_mn_raw")))
        quantize_v_turbo(V.bfloat16(), out=tuple(c[k][l:l + 1] for k in ("V_msb", "V_lsb", "V_scale_turbo")))
        c["Q"][l, :, 0] = q.bfloat16()
    torch.cuda.synchronize()
    return c


def step_bytes(cache, mask, page=64):
    """Algorithmic HBM bytes of one step, each input read once and each output
    written once: scoring = K scale/min of every page; the step's attention
    part = K/V codes + V scale/min of the union of selected pages per KV group,
    plus Q in and O / lse out.  The attention kernel on its own also reads the
    K scale/min of the selected pages (which scoring already counted for the
    step): returned as the third value, the kernel's own algorithmic bytes."""
    L, B, Hkv, P, D = cache["K_scale"].shape
    Hq = cache["Q"].shape[2]
    meta = cache["K_scale"].element_size()
    G = cache["V_scale"].shape[-1]
    scoring = L * B * Hkv * P * D * 2 * meta
    union = mask.view(L, B, Hkv, Hq // Hkv, P).any(3).sum().item()
    per_page = 2 * page * D // 2 + 2 * page * G * meta
    qo = L * B * Hq * (D * 2 * 2 + 4)
    attn_step = union * per_page + qo
    attn_kernel = attn_step + union * 2 * D * meta
    return scoring, attn_step, attn_kernel, union


# --------------------------------------------------------------- measurement --
class Flusher:
    """Evicts L2 (4 MB per XCD) and the 256 MB MALL before each step by reading
    a 1 GiB buffer.  A read leaves clean lines behind; a fill kernel would leave
    up to 256 MB of dirty lines that the timed kernels then have to write back
    (``write=True`` measures that variant, reported as an extra)."""

    def __init__(self, dev, write=False):
        self.buf = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        self.write = write

    def __call__(self):
        if self.write:
            self.buf.fill_(1.0)
        else:
            torch.sum(self.buf)             # one read pass, a 4-byte result


def prefill_inputs(S, Hq, dev, Hkv=8, D=128):
    """A prompt of S tokens written to one layer's INT4 cache (K/V N(0,1) in
    bf16, quantised by this build's quantisers), the bf16 queries, and the
    empty partial-page tail (S is a whole number of pages)."""
    g = torch.Generator(device=dev).manual_seed(7)
    K = torch.randn(1, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    V = torch.randn(1, Hkv, S, D, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(1, Hq, S, D, device=dev, generator=g).to(torch.bfloat16)
    planes = quantize_k_int4(K, 64) + quantize_v_int4(V)
    return q, planes, K[:, :, :0], V[:, :, :0]


def time_steps(fn_pre, fn_timed, steps, warmup, flush, kernel_timer=False):
    """Mean ms of fn_timed over `steps` runs (events on torch's current stream,
    which is the stream the library launches on), each after flush() and the
    untimed fn_pre().  With kernel_timer, also the mean duration of the
    attention kernel alone (library events around each launch)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for _ in range(warmup):
        flush()
        fn_pre()
        fn_timed()
    torch.cuda.synchronize()
    timer = KernelTimer(steps) if kernel_timer else None
    t0 = time.perf_counter()
    if timer:
        timer.__enter__()
    for i in range(steps):
        flush()
        fn_pre()
        ev[i][0].record()
        fn_timed()
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = [a.elapsed_time(b) for a, b in ev]
    kernel_ms = None
    if timer:
        timer.__exit__(None, None, None)
        if timer.launches != steps:
            raise RuntimeError(f"expected {steps} timed attention launches, got {timer.launches}")
        kernel_ms = timer.total_ms / timer.launches
    return sum(ms) / len(ms), wall, kernel_ms


def per_layer_graph_ms(calls, steps, warmup, flush):
    """The reference's per-layer call pattern: `calls` (one decode step per
    layer, in order) captured once in a HIP graph; mean ms per replay."""
    for f in calls:
        f()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for f in calls:
            f()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for f in calls:
                f()
    torch.cuda.synchronize()
    ms, _, _ = time_steps(lambda: None, graph.replay, steps, warmup, flush)
    return ms


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_int4_mfma_config1_traffic.json")


def measured_traffic(L, B, P, retention, select, fused):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (calibrated against a copy of known size),
    when it was measured on this exact workload and kernel; otherwise None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("workload") != {"layers": L, "batch": B, "pages": P, "retention": retention, "select": select,
                              "fused": fused}:
        return None
    return t.get("hbm_bytes_per_launch")


def self_check(cache, dec, mask, k, args):
    """The timed kernel computes the right thing: its in-kernel selection equals
    the selection kernel's (split path) bit for bit on every group, and O of
    every layer agrees with the split path (several workgroups per KV group and
    a merge launch, a different fp32 order) within the north-star 2e-3."""
    from flashquest_amd import _lib as L
    o_fused = dec.O3.clone()
    smask = torch.zeros_like(mask)
    with L.attention_splits(4):
        ref = QuestDecoder(cache["Q"], cache["K_packed"], cache["K_scale"], cache["K_mn"], cache["V_packed"],
                           cache["V_scale"], cache["V_mn"], retention=args.retention, num_sinks=4, window_pages=2,
                           k_max_static=k, select_mode=args.select, mask_out=smask)
        ref()
    torch.cuda.synchronize()
    err = (o_fused.float() - ref.O3.float()).abs().max().item()
    same_sel = bool(torch.equal(mask, smask))
    if not same_sel or not err <= 2e-3 or not torch.isfinite(o_fused).all():
        raise RuntimeError(f"bench self-check failed: selection equal={same_sel}, max|O_fused - O_split|={err}")
    return {"selection_equal_to_split_path": same_sel, "max_abs_O_vs_split_path": err}


def config0(args, dev, flush, noop):
    """Benchmark config 0: one layer, 8k context (128 pages), r = 0.20, the
    benchmark layout (fp16 metadata, V in 32-channel groups), batch 1: the
    whole decode step of one layer (8 KV groups: split over workgroups, the
    split merge), and the CPU baseline on the same layer."""
    from oracle import torch_eager as TE
    c0 = make_cache(1, 1, P=128, dev=dev)
    k0 = math.ceil(0.2 * 128)
    m0 = torch.zeros(1, 1, 24, 128, dtype=torch.bool, device=dev)
    d0 = QuestDecoder(c0["Q"], c0["K_packed"], c0["K_scale"], c0["K_mn"], c0["V_packed"], c0["V_scale"], c0["V_mn"],
                      retention=0.2, num_sinks=4, window_pages=2, k_max_static=k0, select_mode=args.select,
                      mask_out=m0)
    d0()
    torch.cuda.synchronize()
    sb, ab, _, _ = step_bytes(c0, m0)
    d0.mask_out = None
    ms, _, _ = time_steps(noop, d0, args.steps, args.warmup, flush)
    out = {"config0_step_us": ms * 1e3, "config0_step_bytes": sb + ab,
           "config0_step_GBps": (sb + ab) / (ms * 1e-3) / 1e9}
    if not args.no_cpu_baseline:
        threads = max(1, min(16, os.cpu_count() or 1))
        prev = torch.get_num_threads()
        torch.set_num_threads(threads)
        host = {key: v[0, 0].cpu() for key, v in c0.items()}
        times = []
        try:
            for rep in range(12):
                t0 = time.perf_counter()
                o_cpu, sel_cpu = TE.decode_layer(host["Q"][:, 0].float(), host["K_packed"], host["K_scale"],
                                                 host["K_mn"], host["V_packed"], host["V_scale"], host["V_mn"],
                                                 retention=0.2, select=args.select, return_selection=True)
                if rep >= 2:
                    times.append(time.perf_counter() - t0)
        finally:
            torch.set_num_threads(prev)
        out["config0_cpu_baseline_us"] = sorted(times)[len(times) // 2] * 1e6
        out["config0_cpu_threads"] = threads
        out["config0_cpu_check"] = cpu_check(o_cpu[None], sel_cpu[None], d0.O3[0].cpu(), m0[0].cpu())
    return out


def cpu_check(o_cpu, sel_cpu, o_gpu, sel_gpu):
    """The CPU path as the checker of the GPU step on the same layers: how many
    (layer, query head) selections agree (the CPU path scores with torch
    matmuls, the reference's own order), and max |O_gpu - O_cpu| over the
    heads whose selections agree."""
    same = (sel_cpu == sel_gpu).all(-1)                       # (layers, H_q)
    err = (o_gpu.float() - o_cpu).abs().amax(-1)              # (layers, H_q)
    return {"rows": int(same.numel()), "selection_rows_equal": int(same.sum()),
            "max_abs_O_vs_cpu_path": float(err[same].max()) if bool(same.any()) else None}


def sampled_cpu_check(cache, pairs, o_gpu, sel_gpu, retention, select, signs=None):
    """The CPU path (oracle/torch_eager.py) as the checker of a GPU step on a
    sample of (layer, sequence) pairs: o_gpu (L, B, H_q, D), sel_gpu (L, B,
    H_q, P) or None (every page).  With signs (config 3's rotated cache) the
    CPU path rotates q into the cache's basis, x -> WHT(s x) / sqrt(D)
    (Sylvester Hadamard matrix), and O back, y -> s WHT(y) / sqrt(D)."""
    from oracle import torch_eager as TE
    threads = max(1, min(16, os.cpu_count() or 1))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    H = None
    if signs is not None:
        H = torch.ones(1, 1)
        while H.shape[0] < 128:
            H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
        s = signs.float().cpu()
    outs, sels, og, sg = [], [], [], []
    try:
        for l, b in pairs:
            v = {k: cache[k][l, b].cpu() for k in ("Q", "K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")}
            q = v["Q"][:, 0].float()
            if H is not None:
                q = (q * s) @ H / math.sqrt(128)
            o, sel = TE.decode_layer(q, v["K_packed"], v["K_scale"], v["K_mn"], v["V_packed"], v["V_scale"],
                                     v["V_mn"], retention=retention, select=select, return_selection=True)
            if H is not None:
                o = (o @ H / math.sqrt(128)) * s
            outs.append(o)
            sels.append(sel)
            og.append(o_gpu[l, b].float().cpu())
            sg.append(sel if sel_gpu is None else sel_gpu[l, b].cpu())
    finally:
        torch.set_num_threads(prev)
    out = cpu_check(torch.stack(outs), torch.stack(sels), torch.stack(og), torch.stack(sg))
    out["pairs"] = [list(x) for x in pairs]
    return out


def cpu_baseline(cache, args, n_layers, o_gpu, sel_gpu):
    """The reference's eager CPU path restated in PyTorch (oracle/torch_eager.py:
    two fp32 matmuls for the scores, topk + forced pages, fp32 dequant of the
    selected pages, fp32 softmax attention), timed on the host with the box's
    CPU share; median layer time x layers.  Its outputs check the GPU step's
    (o_gpu (L, H_q, D), sel_gpu (L, H_q, P)) on the sampled layers."""
    from oracle import torch_eager as TE
    # a one-GPU box's CPU share is 16 threads (os.cpu_count() there reports the whole host)
    threads = max(1, min(16, os.cpu_count() or 1))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    host = {k: v[:n_layers, 0].cpu() for k, v in cache.items()}
    times, outs, sels = [], [], []
    try:
        for rep in range(2):                               # first pass warms up
            for l in range(n_layers):
                t0 = time.perf_counter()
                o, sel = TE.decode_layer(host["Q"][l, :, 0].float(), host["K_packed"][l], host["K_scale"][l],
                                         host["K_mn"][l], host["V_packed"][l], host["V_scale"][l], host["V_mn"][l],
                                         retention=args.retention, select=args.select, return_selection=True)
                if rep:
                    times.append(time.perf_counter() - t0)
                    outs.append(o)
                    sels.append(sel)
    finally:
        torch.set_num_threads(prev)
    per_layer = sorted(times)[len(times) // 2]
    check = cpu_check(torch.stack(outs), torch.stack(sels), o_gpu[:n_layers].cpu(), sel_gpu[:n_layers].cpu())
    return {"value": per_layer * args.layers * 1e6, "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{n_layers} layers of the same workload (batch 1), median layer time x {args.layers}; "
                      f"eager PyTorch restatement of the reference CPU path, {threads} threads",
            "check": check}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is design-only",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L, B, P = args.layers, args.batch, args.pages
    if args.profile_int8:
        from flashquest_amd.eager.decode import quest_decode_int8
        ic = make_int8_cache(L, P=P, dev=dev)
        iplanes = [ic[x] for x in ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")]
        flush = Flusher(dev)
        k = math.ceil(args.retention * P)
        for _ in range(10):
            flush()
            quest_decode_int8(ic["Q"], *iplanes, retention=args.retention, num_sinks=4, window_pages=2,
                              k_max_static=k, select_mode=args.select)
        torch.cuda.synchronize()
        print(json.dumps({"profile_int8": "done", "select": args.select}))
        return
    if args.profile_prefill:
        from flashquest_amd.kernel import flash_attn_prefill_int4
        qp, pk, kt, vt = prefill_inputs(P * 64, 24, dev)   # config 1 shape: 24 query / 8 KV heads
        for _ in range(8):       # the first 3 bring the GPU clock up; the last 5 are the ones reported
            flash_attn_prefill_int4(qp, *pk, kt, vt, page_size=64)
        torch.cuda.synchronize()
        print(json.dumps({"profile_prefill": "done", "tokens": P * 64}))
        return
    if args.profile_turbo:
        from flashquest_amd.eager.decode import quest_decode_turbo
        tc = make_turbo_cache(L, P=P, dev=dev)
        planes = [tc[x] for x in ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")]
        flush = Flusher(dev)
        k = math.ceil(args.retention * P)
        for _ in range(10):
            flush()
            quest_decode_turbo(tc["Q"], *planes, tc["K_scale_raw"], tc["K_mn_raw"], retention=args.retention,
                               num_sinks=4, window_pages=2, k_max_static=k, select_mode=args.select)
        torch.cuda.synchronize()
        print(json.dumps({"profile_turbo": "done", "select": args.select}))
        return

    cache = make_cache(L, B, P=P, dev=dev)
    Hq = cache["Q"].shape[2]
    flush = Flusher(dev)
    k = math.ceil(args.retention * P)

    def decoder(retention, kmax, mode, c=cache, mask=None):
        return QuestDecoder(c["Q"], c["K_packed"], c["K_scale"], c["K_mn"], c["V_packed"], c["V_scale"], c["V_mn"],
                            retention=retention, num_sinks=4, window_pages=2, k_max_static=kmax,
                            select_mode=mode, mask_out=mask)

    if args.profile_per_layer:
        per_layer = [decoder(args.retention, k, args.select,
                             c={key: t[l] for key, t in cache.items()}) for l in range(L)]
        per_layer_graph_ms(per_layer, 5, 1, flush)
        torch.cuda.synchronize()
        print(json.dumps({"profile_per_layer": "done", "select": args.select}))
        return

    if args.profile_gqa8:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)                      # FETCH = WRITE = 256 MiB of HBM traffic
        c8 = make_cache(L, B, Hq=64, P=P, dev=dev)
        dec = decoder(args.retention, k, args.select, c=c8)
        for _ in range(5):
            flush()
            dec()
        torch.cuda.synchronize()
        print(json.dumps({"profile_gqa8": "done", "select": args.select, "copy_bytes": src.numel()}))
        return

    if args.profile_kernels:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)                      # FETCH = WRITE = 256 MiB of HBM traffic
        dec = decoder(args.retention, k, args.select)
        for _ in range(3):
            flush()
            dec()
        torch.cuda.synchronize()
        print(json.dumps({"profile_kernels": "done", "copy_bytes": src.numel()}))
        return

    mask = torch.zeros(L, B, Hq, P, dtype=torch.bool, device=dev)
    dec = decoder(args.retention, k, args.select, mask=mask)
    dec()
    torch.cuda.synchronize()
    scoring_b, attn_b, attn_kernel_b, union = step_bytes(cache, mask)
    dec.mask_out = None
    noop = lambda: None
    check = self_check(cache, dec, mask, k, args)
    step_ms, wall, _ = time_steps(noop, dec, args.steps, args.warmup, flush)
    attend_ms, _, attn_ms = time_steps(dec.select, dec.attend, args.steps, args.warmup, flush, kernel_timer=True)
    total_b = scoring_b + attn_b
    # the access pattern's ceiling: the same bytes read in the same order with no compute
    planes = [cache[x] for x in ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")]
    rd_ms, _, rd_kernel_ms = time_steps(noop, lambda: read_decode_pages(*planes, mask), args.steps, args.warmup, flush,
                                        kernel_timer=True)
    # the plainest read of the same byte count: one contiguous buffer, no pattern
    sbuf = torch.empty((total_b + 15) // 16 * 16, dtype=torch.uint8, device=dev)
    _, _, st_kernel_ms = time_steps(noop, lambda: read_stream(sbuf), args.steps, args.warmup, flush, kernel_timer=True)
    del sbuf
    extra = {"self_check": check, "union_pages_per_kv_head": union / (L * B * 8), "step_bytes": total_b,
             "step_GBps": total_b / (step_ms * 1e-3) / 1e9,
             "step_roofline_frac": total_b / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
             "attention_kernel_us": attn_ms * 1e3, "attend_with_split_merge_us": attend_ms * 1e3,
             "select_us": None, "select_mode": args.select,
             # the read-only kernel alone (library events around its launch), and the
             # probe call's time with its union-list launch
             "read_only_kernel_us": rd_kernel_ms * 1e3,
             "read_only_kernel_roofline_frac": total_b / (rd_kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
             "attention_kernel_over_read_only_kernel": attn_ms / rd_kernel_ms,
             "stream_read_kernel_us": st_kernel_ms * 1e3,
             "stream_read_GBps": total_b / (st_kernel_ms * 1e-3) / 1e9,
             "attention_kernel_over_stream_read": attn_ms / st_kernel_ms,
             "read_only_pass_with_union_us": rd_ms * 1e3}
    if not args.no_extra:
        extra.update(config0(args, dev, flush, noop))
        ctl = decoder(1.0, P, args.select)
        ctl_ms, _, _ = time_steps(noop, ctl, args.steps, args.warmup, flush)
        full_mask = torch.ones(L, B, Hq, P, dtype=torch.bool, device=dev)
        sb, ab, _, _ = step_bytes(cache, full_mask)
        extra.update({"all_pages_control_us": ctl_ms * 1e3, "sparse_speedup_vs_all_pages": ctl_ms / step_ms,
                      "all_pages_GBps": (sb + ab) / (ctl_ms * 1e-3) / 1e9})
        if not args.no_cpu_baseline:
            ctl()
            torch.cuda.synchronize()
            extra["config2_cpu_check"] = sampled_cpu_check(cache, [(0, 0), (13, 0), (27, 0)][:L], ctl.O3, None, 1.0,
                                                           args.select)
        other = "per_q_head" if args.select == "per_kv_head_sum" else "per_kv_head_sum"
        alt = decoder(args.retention, k, other)
        alt_ms, _, _ = time_steps(noop, alt, args.steps, args.warmup, flush)
        extra[f"{other}_us"] = alt_ms * 1e3
        # 8 query heads per KV head (64 query / 8 KV heads, the Llama-3-70B
        # layout) on otherwise the same synthetic layers: the query heads of a
        # group in two chunks of 4 on the matrix-core kernels
        c8 = make_cache(L, B, Hq=64, P=P, dev=dev)
        for mode in ("per_kv_head_sum", "per_q_head"):
            d8 = decoder(args.retention, k, mode, c=c8)
            ms8, _, _ = time_steps(noop, d8, args.steps, args.warmup, flush)
            extra[f"gqa8_{mode}_us"] = ms8 * 1e3
        del c8, d8
        # the reference's per-layer call pattern: 28 sequential (select, attend) pairs in one HIP graph
        per_layer = [decoder(args.retention, k, args.select,
                             c={key: t[l] for key, t in cache.items()}) for l in range(L)]
        extra["per_layer_graph_us"] = per_layer_graph_ms(per_layer, args.steps, args.warmup, flush) * 1e3
        # the same pattern issued eagerly through the functional operator (the
        # reference patch's call, new output tensors every layer): host-side
        # cost included
        from flashquest_amd.eager.decode import quest_decode_int4 as _qd4
        lviews = [[cache[x][l] for x in ("Q", "K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")]
                  for l in range(L)]

        def eager_layers():
            for v in lviews:
                _qd4(v[0], *v[1:], retention=args.retention, num_sinks=4, window_pages=2, k_max_static=k,
                     select_mode=args.select)
        eager_ms, _, _ = time_steps(noop, eager_layers, args.steps, args.warmup, flush)
        extra["per_layer_eager_us"] = eager_ms * 1e3
        del lviews
        # the same, with a 37-token bf16 partial page per layer (the usual decode
        # step): the tail is attended in the split-merge launch
        T_tail = 37
        kt = torch.randn(L, B, 8, T_tail, 128, device=dev).bfloat16()
        vt = torch.randn(L, B, 8, T_tail, 128, device=dev).bfloat16()
        tdec = QuestDecoder(cache["Q"], cache["K_packed"], cache["K_scale"], cache["K_mn"], cache["V_packed"],
                            cache["V_scale"], cache["V_mn"], retention=args.retention, num_sinks=4, window_pages=2,
                            k_max_static=k, select_mode=args.select, K_tail=kt, V_tail=vt)
        tt_ms, _, _ = time_steps(noop, tdec, args.steps, args.warmup, flush)
        extra["step_with_tail_us"] = tt_ms * 1e3
        per_layer_t = [QuestDecoder(*[cache[key][l] for key in ("Q", "K_packed", "K_scale", "K_mn", "V_packed",
                                                                "V_scale", "V_mn")], retention=args.retention,
                                    num_sinks=4, window_pages=2, k_max_static=k, select_mode=args.select,
                                    K_tail=kt[l], V_tail=vt[l]) for l in range(L)]
        extra["per_layer_graph_with_tail_us"] = per_layer_graph_ms(per_layer_t, args.steps, args.warmup, flush) * 1e3
        del kt, vt, tdec, per_layer_t
        sel_ms, _, _ = time_steps(noop, dec.select, args.steps, args.warmup, flush)
        extra["select_us"] = sel_ms * 1e3 if not dec.fused else None
        wflush = Flusher(dev, write=True)
        wf_ms, _, _ = time_steps(noop, dec, args.steps, args.warmup, wflush)
        extra["step_us_after_write_flush"] = wf_ms * 1e3
        del wflush

        # benchmark config 3: rotated INT4 (K, V rotated by x -> WHT(s x) / sqrt(128)
        # before quantisation).  The single launch rotates Q in its prologue and
        # O back in its store.
        signs = rotation_signs(dev=dev)
        rc = make_cache(L, B, P=P, dev=dev, signs=signs)
        from flashquest_amd.eager.decode import quest_decode_int4
        rplanes = [rc[x] for x in ("K_packed", "K_scale", "K_mn", "V_packed", "V_scale", "V_mn")]
        _, _, rmask = quest_decode_int4(rc["Q"], *rplanes, retention=args.retention, num_sinks=4, window_pages=2,
                                        k_max_static=k, select_mode=args.select, return_selection=True,
                                        rotation_signs=signs)      # the kernel's own selection, as a mask
        rdec = QuestDecoder(rc["Q"], *rplanes, retention=args.retention, num_sinks=4, window_pages=2,
                            k_max_static=k, select_mode=args.select, rotation_signs=signs)
        torch.cuda.synchronize()
        rs_b, ra_b, _, _ = step_bytes(rc, rmask)
        r_ms, _, _ = time_steps(noop, rdec, args.steps, args.warmup, flush)
        if not args.no_cpu_baseline:
            rdec()
            torch.cuda.synchronize()
            extra["config3_cpu_check"] = sampled_cpu_check(rc, [(0, 0), (13, 0), (27, 0)][:L], rdec.O3, rmask,
                                                           args.retention, args.select, signs=signs)
        extra.update({"config3_rotated_us": r_ms * 1e3, "config3_fused": rdec.fused,
                      "config3_step_GBps": (rs_b + ra_b) / (r_ms * 1e-3) / 1e9,
                      "config3_roofline_frac": (rs_b + ra_b) / (r_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                      "config3_over_config1": r_ms / step_ms})
        del rc, rdec, rmask

        # TurboQuant K3-V3 (the reference's kv_bits == 3 path) over all layers:
        # the fused decode (scores from the raw K page metadata, selection,
        # turbo attention) in both selection modes, and the reference's operator
        # sequence (page scores, per-query-head top-k, mask attention)
        from flashquest_amd.eager.criticality import page_scores_int4_fast
        from flashquest_amd.eager.decode import quest_decode_turbo
        from flashquest_amd.eager.selection import select_pages_vectorized
        from flashquest_amd.kernel.sparse_turbo_fwd import flash_attn_sparse_turbo_fwd
        tc = make_turbo_cache(L, P=P, dev=dev)
        planes = [tc[x] for x in ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo")]

        def turbo_bytes(mask):
            union = mask.view(L, 8, Hq // 8, P).any(2).sum().item()
            return (L * 8 * P * 128 * 2 * 2 + union * 64 * (2 * (16 + 32) + 2 * 2) + L * Hq * (128 * 2 * 2 + 4)), union

        for mode in ("per_kv_head_sum", "per_q_head"):
            _, _, tmask = quest_decode_turbo(tc["Q"], *planes, tc["K_scale_raw"], tc["K_mn_raw"], retention=args.retention,
                                             num_sinks=4, window_pages=2, k_max_static=k, select_mode=mode,
                                             return_selection=True)
            torch.cuda.synchronize()
            t_bytes, t_union = turbo_bytes(tmask)
            t_ms, _, _ = time_steps(noop, lambda: quest_decode_turbo(
                tc["Q"], *planes, tc["K_scale_raw"], tc["K_mn_raw"], retention=args.retention, num_sinks=4,
                window_pages=2, k_max_static=k, select_mode=mode), args.steps, args.warmup, flush)
            extra.update({f"turbo_{mode}_us": t_ms * 1e3, f"turbo_{mode}_union_pages_per_kv_head": t_union / (L * 8),
                          f"turbo_{mode}_step_GBps": t_bytes / (t_ms * 1e-3) / 1e9,
                          f"turbo_{mode}_roofline_frac": t_bytes / (t_ms * 1e-3) / 1e9 / HBM_PEAK_GBS})
            tkeys = ("K_msb", "K_lsb", "K_scale_turbo", "V_msb", "V_lsb", "V_scale_turbo", "K_scale_raw", "K_mn_raw")
            calls = [(lambda l=l: quest_decode_turbo(tc["Q"][l:l + 1], *[tc[x][l:l + 1] for x in tkeys],
                                                     retention=args.retention, num_sinks=4, window_pages=2,
                                                     k_max_static=k, select_mode=mode)) for l in range(L)]
            extra[f"turbo_{mode}_per_layer_graph_us"] = per_layer_graph_ms(calls, args.steps, args.warmup, flush) * 1e3

        def turbo_ops_step():
            sc = page_scores_int4_fast(tc["Q"], tc["K_scale_raw"], tc["K_mn_raw"])
            m = select_pages_vectorized(sc, args.retention, 4, 2, k_max_static=k)
            return flash_attn_sparse_turbo_fwd(tc["Q"], *planes, selection_mask=m)[0]

        t_ms, _, _ = time_steps(noop, turbo_ops_step, args.steps, args.warmup, flush)
        extra["turbo_reference_operator_sequence_us"] = t_ms * 1e3
        del tc, planes

        # INT8 KV (the reference dispatcher's default kv_bits = 8): score
        # (255 levels) -> select -> flash_attn_sparse_fwd over all layers
        from flashquest_amd.eager.decode import quest_decode_int8
        ic = make_int8_cache(L, P=P, dev=dev)
        iplanes = [ic[x] for x in ("K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")]
        _, _, imask = quest_decode_int8(ic["Q"], *iplanes, retention=args.retention, num_sinks=4, window_pages=2,
                                        k_max_static=k, select_mode=args.select, return_selection=True)
        torch.cuda.synchronize()
        i_union = imask.view(L, 8, Hq // 8, P).any(2).sum().item()
        i_bytes = L * 8 * P * 128 * 2 * 2 + i_union * 64 * (2 * 128 + 2 * 2) + L * Hq * (128 * 2 * 2 + 4)
        i_ms, _, _ = time_steps(noop, lambda: quest_decode_int8(
            ic["Q"], *iplanes, retention=args.retention, num_sinks=4, window_pages=2, k_max_static=k,
            select_mode=args.select), args.steps, args.warmup, flush)
        extra.update({"int8_us": i_ms * 1e3, "int8_step_bytes": i_bytes,
                      "int8_step_GBps": i_bytes / (i_ms * 1e-3) / 1e9,
                      "int8_roofline_frac": i_bytes / (i_ms * 1e-3) / 1e9 / HBM_PEAK_GBS})
        ikeys = ("Q", "K_uint8", "K_scale", "K_mn", "V_uint8", "V_scale", "V_mn")
        calls = [(lambda l=l: quest_decode_int8(*[ic[x][l:l + 1] for x in ikeys], retention=args.retention,
                                                num_sinks=4, window_pages=2, k_max_static=k,
                                                select_mode=args.select)) for l in range(L)]
        extra["int8_per_layer_graph_us"] = per_layer_graph_ms(calls, args.steps, args.warmup, flush) * 1e3
        kt8 = torch.randn(L, 8, 37, 128, device=dev).bfloat16()      # a 37-token partial page per layer
        vt8 = torch.randn(L, 8, 37, 128, device=dev).bfloat16()
        calls = [(lambda l=l: quest_decode_int8(*[ic[x][l:l + 1] for x in ikeys], retention=args.retention,
                                                num_sinks=4, window_pages=2, k_max_static=k, select_mode=args.select,
                                                K_tail=kt8[l:l + 1], V_tail=vt8[l:l + 1])) for l in range(L)]
        extra["int8_per_layer_graph_with_tail_us"] = per_layer_graph_ms(calls, args.steps, args.warmup, flush) * 1e3
        del kt8, vt8
        del ic, iplanes

        # Prefill over the packed cache (the reference's S_q > 1 branch,
        # llama_persistent_patch.py:196-201) for one layer and a 32k-token
        # prompt already written to the INT4 cache: this build's kernel
        # (dequantise once, causal bf16 flash attention on the matrix cores) vs
        # the reference's operator sequence (dequantise with tensor ops,
        # concatenate, SDPA is_causal) timed on the same GPU.
        from flashquest_amd.kernel import dequantize_k_int4, dequantize_v_int4, flash_attn_prefill_int4
        import torch.nn.functional as F
        Sp = P * 64
        qp, pk, kt, vt = prefill_inputs(Sp, Hq, dev)
        pf_steps = max(3, args.steps // 4)
        pf_ms, _, _ = time_steps(noop, lambda: flash_attn_prefill_int4(qp, *pk, kt, vt, page_size=64),
                                 pf_steps, 1, noop)

        def ref_prefill():
            Kf = torch.cat([dequantize_k_int4(pk[0], pk[1], pk[2], 64), kt], dim=2)
            Vf = torch.cat([dequantize_v_int4(pk[3], pk[4], pk[5]), vt], dim=2)
            return F.scaled_dot_product_attention(qp, Kf, Vf, is_causal=True, enable_gqa=True)
        pr_ms, _, _ = time_steps(noop, ref_prefill, pf_steps, 1, noop)
        # a 128-token chunk over the same cache, lower-right aligned (key-range splits)
        qc = qp[:, :, -128:].contiguous()
        pc_ms, _, _ = time_steps(noop, lambda: flash_attn_prefill_int4(qc, *pk, kt, vt, page_size=64,
                                                                       causal_offset=Sp - 128), pf_steps, 1, noop)
        extra["prefill_chunk128_over_32k_us"] = pc_ms * 1e3
        pf_flops = 2.0 * Sp * Sp * 128 * Hq          # causal: 4 S^2 D H_q / 2
        extra.update({"prefill_32k_layer_ms": pf_ms, "prefill_TFLOPs": pf_flops / (pf_ms * 1e-3) / 1e12,
                      "prefill_mfma_frac": pf_flops / (pf_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                      "prefill_reference_sequence_ms": pr_ms, "prefill_speedup_vs_reference_sequence": pr_ms / pf_ms})
        del qp, pk

        # benchmark config 4: batch 16 independent sequences, 28 layers, 32k each
        if B == 1 and args.batch16:
            bc = make_cache(L, 16, P=P, dev=dev)
            bmask = torch.zeros(L, 16, Hq, P, dtype=torch.bool, device=dev)
            bdec = decoder(args.retention, k, args.select, c=bc, mask=bmask)
            bdec()
            torch.cuda.synchronize()
            bs_b, ba_b, _, _ = step_bytes(bc, bmask)
            bdec.mask_out = None
            b_ms, _, _ = time_steps(noop, bdec, args.steps, args.warmup, flush)
            if not args.no_cpu_baseline:
                bdec()
                torch.cuda.synchronize()
                extra["config4_cpu_check"] = sampled_cpu_check(bc, [(0, 0), (5, 7), (13, 15), (27, 3)], bdec.O3,
                                                               bmask, args.retention, args.select)
            extra.update({"config4_batch16_us": b_ms * 1e3, "config4_step_bytes": bs_b + ba_b,
                          "config4_step_GBps": (bs_b + ba_b) / (b_ms * 1e-3) / 1e9,
                          "config4_roofline_frac": (bs_b + ba_b) / (b_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "config4_fused": bdec.fused})
            del bc, bdec, bmask

    # The dominant kernel: with one workgroup per KV group the attention kernel
    # scores and selects its own pages, so one launch is the whole step and its
    # algorithmic bytes are the step's (every page's K scale/min once, the
    # selected pages' codes and V scale/min, Q, O, lse).  Otherwise the
    # attention kernel alone, which also reads the selected pages' K scale/min.
    fused = dec.fused
    kernel_b = scoring_b + attn_b if fused else attn_kernel_b
    kname = ("attn_int4_mfma_kernel, fused: score + select + sparse attention for all layers in one launch"
             if fused else "attn_int4_mfma_kernel (sparse GQA attention, all layers in one launch)")
    traffic = measured_traffic(L, B, P, args.retention, args.select, fused)
    roof = {"bound": "hbm", "achieved": kernel_b / (attn_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": kernel_b / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "traffic": traffic,
            "kernel": kname, "kernel_us": attn_ms * 1e3, "algorithmic_bytes_per_launch": kernel_b}
    cpu = None
    if not args.no_cpu_baseline and B == 1:
        dec()                       # the timed step's output (deterministic) for the check
        torch.cuda.synchronize()
        cpu = cpu_baseline(cache, args, min(args.cpu_layers, L), dec.O3[:, 0], mask[:, 0])
    line = {
        "metric": METRIC, "value": step_ms * 1e3, "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": step_ms, "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 KV; q.k on int8 MFMA (exact 3-digit split of q*K_scale, int32 accumulate); p.v on fp16 MFMA "
                 "with p*V_scale as fp16 hi + lo parts (fp32-level operand, 2^-22 relative) times the exact INT4 "
                 "codes, fp32 accumulate; fp32 softmax; fp16 output",
        "data": "synthetic",
        "config": {"workload": f"BASELINE config 1: {L} independent layers x batch {B}, {Hq}/8 heads, D=128, "
                               f"{P} pages x 64 tokens, retention {args.retention} ({args.select} top-{k} + 4 sink "
                               "+ 2 window pages), INT4 K/V with fp16 metadata (V per 32 channels), "
                               "L2/MALL flushed between steps",
                   "layers": L, "batch": B, "context": P * 64, "retention": args.retention},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra, "wall_s_timed_region": wall,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
