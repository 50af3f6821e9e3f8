"""The public API's fast path and the packed-varlen layout (GPU).

flash_attn_with_kvcache sends the common decode call (one token, a paged
16-bit cache, int32 metadata, default options) straight to the C++ operator.
It must return what the full path returns, bit for bit (the same kernels),
record the same dispatch information, and leave every other call, valid or
not, to the full path: the same routes, errors and messages.
"""

from __future__ import annotations

import pytest
import torch

import mxflashattn_amd as mx
from mxflashattn_amd import native
from mxflashattn_amd.integrations.vllm import decode_step
from mxflashattn_amd.workloads import make_paged_batch
from oracle import reference_port

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def api(b, **kw):
    return mx.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, cache_seqlens=b.cache_seqlens,
                                      block_table=b.block_table, **kw)


def full_path(b, monkeypatch, **kw):
    """The same call with the fast path switched off (strict validation on
    also reads the lengths back, which changes nothing for valid inputs)."""
    with monkeypatch.context() as m:
        m.setenv("MXFLASHATTN_STRICT_VALIDATION", "1")
        return api(b, **kw)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("hq,hkv,hd", [(32, 8, 128), (16, 8, 64), (32, 4, 64), (32, 32, 128)])
def test_fast_path_equals_full_path(device, monkeypatch, dtype, hq, hkv, hd):
    g = torch.Generator().manual_seed(hq + hd)
    b = make_paged_batch(9, hq, hkv, hd, dtype, torch.randint(1, 3000, (9,), generator=g),
                         seed=hd + hkv).to(device)
    fast = api(b)
    info = mx.get_last_dispatch_info()
    assert info.backend == mx.BACKEND_MI355X and info.operation == "flash_attn_with_kvcache"
    assert info.fallback_reason is None
    slow = full_path(b, monkeypatch)
    torch.cuda.synchronize()
    assert torch.isfinite(fast.float()).all()
    assert torch.equal(fast, slow)
    assert mx.get_last_dispatch_info() == info
    # out= is written and returned; an explicit scale equals the default one.
    out = torch.full_like(b.q, float("nan"))
    got = api(b, out=out, softmax_scale=float(hd ** -0.5))
    torch.cuda.synchronize()
    assert got is out and torch.equal(out, fast)
    cpu = b.to("cpu")
    want = reference_port.attention_kvcache(cpu.q, cpu.k_cache, cpu.v_cache,
                                            cache_seqlens=cpu.cache_seqlens.clone(),
                                            block_table=cpu.block_table, softmax_scale=cpu.scale)
    assert (fast.float().cpu() - want.float()).abs().max().item() <= TOL[dtype]


def test_fast_path_leaves_other_calls_to_the_full_path(device):
    b = make_paged_batch(4, 16, 4, 128, torch.bfloat16, torch.tensor([3, 70, 200, 5]),
                         seed=5).to(device)
    # Head dim 256 is outside the reference's API contract: the full path's message.
    b256 = make_paged_batch(2, 8, 2, 256, torch.bfloat16, torch.tensor([3, 9]), seed=6).to(device)
    with pytest.raises(ValueError, match="head dimension must be 64 or 128"):
        api(b256)
    # int64 lengths: not the operator's call; the full path converts and decodes.
    got = mx.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache,
                                     cache_seqlens=b.cache_seqlens.long(),
                                     block_table=b.block_table)
    assert torch.equal(got, api(b))
    # A wrong out, an overlapping out, options the API rejects: full-path errors.
    with pytest.raises(ValueError, match="out must match"):
        api(b, out=torch.empty(4, 1, 16, 64, device=device, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="overlapping"):
        api(b, out=torch.empty(1, 1, 16, 128, device=device,
                               dtype=torch.bfloat16).expand(4, 1, 16, 128))
    with pytest.raises(NotImplementedError, match="soft-capping"):
        api(b, softcap=5.0)
    with pytest.raises(ValueError, match="finite"):
        api(b, softmax_scale=float("inf"))
    with pytest.raises(ValueError, match="cache_seqlens must be one-dimensional"):
        mx.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache,
                                   cache_seqlens=b.cache_seqlens[:3], block_table=b.block_table)
    torch.cuda.synchronize()


def test_packed_varlen_layout_equals_varlen_api(device):
    """The bench's packed layout (one-token pages, table row = offset +
    arange) is what flash_attn_varlen_func decode builds from cu_seqlens_k."""
    lens = torch.tensor([700, 1, 2300, 64, 0, 1500])
    b = make_paged_batch(6, 32, 8, 128, torch.bfloat16, lens, page_size=1, packed=True,
                         seed=9).to(device)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, out=torch.full_like(b.q, float("nan")))
    keep = lens > 0  # the varlen API requires keys for every sequence it is given
    cu = torch.zeros(int(keep.sum()) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens[keep], 0)
    cu_q = torch.arange(int(keep.sum()) + 1, dtype=torch.int32)
    k = b.k_cache[:, 0]  # [total_tokens, HKV, HD]
    v = b.v_cache[:, 0]
    ref = mx.flash_attn_varlen_func(b.q[keep.to(device), 0], k, v, cu_q.to(device), cu.to(device),
                                    1, int(lens.max()))
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got[keep.to(device), 0], ref)
    assert torch.equal(got[4], torch.zeros_like(got[4]))  # the empty sequence


def test_eager_decode_step_runs(device):
    shape = decode_step.DecoderShape(layers=2, hidden=256, q_heads=8, kv_heads=2, head_dim=128,
                                     intermediate=512, vocab=1000)
    res = decode_step.run(batch=4, new_tokens=6, shape=shape, median=64, lo=16, hi=256,
                          device=device, eager=True)
    assert res["mode"] == "eager" and res["logits_finite"]
    assert res["step_ms"] > 0 and 0 < res["attention_share"] <= 1.5
    assert res["attention_host_us_per_layer"] > 0 and res["timed_steps"] == 5


def test_reshape_and_cache_operator_equals_ctypes_path(device, monkeypatch):
    """The vLLM-form append through the C++ operator and through ctypes write
    the same bytes; slots < 0 are skipped by both."""
    g = torch.Generator().manual_seed(17)
    pages, ps, hkv, hd = 40, 16, 8, 128
    key = torch.randn(50, hkv, hd, generator=g).to(torch.bfloat16)
    value = torch.randn(50, hkv, hd, generator=g).to(torch.bfloat16)
    slots = torch.randperm(pages * ps, generator=g)[:50]
    slots[[3, 17]] = -1
    caches = []
    for use_op in (True, False):
        monkeypatch.setattr(native, "USE_TORCH_OP", use_op)
        kc = torch.zeros(pages, ps, hkv, hd, dtype=torch.bfloat16, device=device)
        vc = torch.zeros_like(kc)
        native.reshape_and_cache(key.to(device), value.to(device), kc, vc, slots.to(device))
        caches.append((kc, vc))
    torch.cuda.synchronize()
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    kc = caches[0][0].cpu().view(pages * ps, hkv, hd)
    keep = slots >= 0
    assert torch.equal(kc[slots[keep]], key[keep])
    assert int((kc.abs().sum((1, 2)) > 0).sum()) == int(keep.sum())
