"""Host side of the prefill operators on the CPU: no CPU fallback (device
tensors are required, as for every operator of this build), the C ABI's
argument checks and workspace sizing, without launching anything."""
import ctypes

import pytest
import torch

from flashquest_amd import _lib as L


def _cache(S=256, P=4, D=128, Hkv=2, L_=1):
    c = L.Int4Cache()
    c.k_packed = c.v_packed = c.k_scale = c.k_mn = c.v_scale = c.v_mn = 4096
    c.k_strides = L.i64([0, Hkv * S * D // 2, S * D // 2, D // 2, 1], 5)
    c.v_strides = L.i64([0, Hkv * S * D // 2, S * D // 2, D // 2, 1], 5)
    c.ks_strides = c.km_strides = L.i64([0, Hkv * P * D, P * D, D, 1], 5)
    c.vs_strides = c.vm_strides = L.i64([0, Hkv * S, S, 1, 1], 5)
    c.meta_dtype = L.FQ_BF16
    c.L, c.B, c.H_kv, c.S, c.P, c.D, c.page_size, c.v_groups = L_, 1, Hkv, S, P, D, 64, 1
    return c


def _query(Sq, Hq=6, off=0, D=128):
    q = L.Prefill()
    q.q = q.out = 8192
    q.q_strides = q.o_strides = L.i64([Hq * Sq * D, Sq * D, D, 1], 4)
    q.H_q, q.S_q, q.causal_offset, q.sm_scale, q.D = Hq, Sq, off, 0.0, D
    return q


def test_prefill_requires_device_tensors():
    from flashquest_amd.kernel import flash_attn_prefill_int4
    q = torch.zeros(1, 6, 4, 128, dtype=torch.bfloat16)
    kp = torch.zeros(1, 2, 64, 64, dtype=torch.uint8)
    meta = torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16)
    vmeta = torch.zeros(1, 2, 64, 1, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        flash_attn_prefill_int4(q, kp, meta, meta, kp, vmeta, vmeta, page_size=64)


def test_prefill_workspace_sizing():
    lib = L.lib()
    tail = L.Tail()
    # one row block over few keys: the kernel dequantises its own tiles, no workspace
    assert lib.fq_prefill_workspace_bytes(_cache(S=256), tail, _query(Sq=40), 4) == 0
    # a long prompt: dense bf16 K and V^T, 512 B per attended key and KV head (keys rounded to 128)
    assert lib.fq_prefill_workspace_bytes(_cache(S=256), tail, _query(Sq=256), 4) == 2 * 256 * 512
    # invalid arguments report 0 (the call itself then reports the error)
    assert lib.fq_prefill_workspace_bytes(_cache(S=256), tail, _query(Sq=256, Hq=5), 4) == 0
    assert lib.fq_prefill_workspace_bytes(_cache(S=256, D=64), tail, _query(Sq=256, D=64), 4) == 0


def test_prefill_argument_errors():
    lib = L.lib()
    tail = L.Tail()
    cases = [(_cache(L_=2), _query(Sq=8), L.FQ_ERR_INVALID),            # more than one layer
             (_cache(D=64), _query(Sq=8, D=64), L.FQ_ERR_UNSUPPORTED),  # head_dim 64
             (_cache(), _query(Sq=8, Hq=5), L.FQ_ERR_INVALID),          # H_q not a multiple of H_kv
             (_cache(), _query(Sq=8, off=-1), L.FQ_ERR_INVALID),        # negative causal offset
             (_cache(), _query(Sq=0), L.FQ_ERR_INVALID),                # no queries
             (_cache(), _query(Sq=8, D=64), L.FQ_ERR_INVALID)]          # q head_dim != the cache's
    for c, q, want in cases:
        assert lib.fq_prefill_int4(c, tail, q, None, 0, None) == want
    # a long prompt without its workspace
    assert lib.fq_prefill_int4(_cache(), tail, _query(Sq=256), None, 0, None) == L.FQ_ERR_WORKSPACE
