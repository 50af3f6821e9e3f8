"""The vLLM backend classes (integrations/vllm/vllm_plugin.py) against a
stand-in for vLLM's FlashAttention module, since vLLM is not installed.

The reference's tests/test_vllm_official_split_fallback.py skips without vLLM;
here the stand-in's ``FlashAttentionImpl.forward`` calls whatever
``flash_attn_with_kvcache`` its module globals hold at call time, as vLLM's
does, so the swap, the retry and the restore are observable."""

import importlib
import sys
import types

import pytest
import torch

from mxflashattn_amd.integrations.vllm import backend, native_decode
from mxflashattn_amd.integrations.vllm.decoder_adapter import DecoderAdapterBlocked

PLUGIN = "mxflashattn_amd.integrations.vllm.vllm_plugin"
FA = "vllm.v1.attention.backends.flash_attn"

_FAKE_FLASH_ATTN = '''
def flash_attn_with_kvcache(*args, **kwargs):
    return "vendor_kvcache"

class FlashAttentionImpl:
    def __init__(self, attn_type="decoder", kv_cache_dtype="auto"):
        self.scale = 0.125
        self.attn_type = attn_type
        self.kv_cache_dtype = kv_cache_dtype

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        return flash_attn_with_kvcache(query, kv_cache)

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        return "vendor_cache_update"

class FlashAttentionBackend:
    pass
'''


@pytest.fixture
def plugin(monkeypatch):
    fa = types.ModuleType(FA)
    exec(_FAKE_FLASH_ATTN, fa.__dict__)
    for name in ("vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, FA, fa)
    monkeypatch.delitem(sys.modules, PLUGIN, raising=False)
    for var in ("MXFLASHATTN_SPLIT_PURE", "MXFLASHATTN_GRAPH_OFFICIAL_SPLIT",
                "MXFA_WIDE_CONTRACT"):
        monkeypatch.delenv(var, raising=False)
    backend.clear_dispatch_events(truncate_log=False)
    mod = importlib.import_module(PLUGIN)
    yield mod, fa
    sys.modules.pop(PLUGIN, None)
    pkg = sys.modules["mxflashattn_amd.integrations.vllm"]
    if hasattr(pkg, "vllm_plugin"):
        delattr(pkg, "vllm_plugin")


def _forward(mod, impl=None, metadata="meta", output="out", layer=None):
    impl = impl or mod.MXFlashAttnImpl()
    return impl.forward(layer, "q", "k", "v", "kv_cache", metadata, output)


def test_backend_names_the_flash_attn_slot(plugin):
    mod, _ = plugin
    assert mod.MXFlashAttnBackend.get_name() == "FLASH_ATTN"
    assert mod.MXFlashAttnBackend.get_impl_cls() is mod.MXFlashAttnImpl


def test_official_split_swaps_kvcache_for_the_call_only(plugin, monkeypatch):
    mod, fa = plugin
    vendor = fa.flash_attn_with_kvcache
    seen = {}

    def compat(*args, **kwargs):
        seen["official"] = native_decode.official_kvcache
        return "mx_kvcache"

    monkeypatch.setattr(native_decode, "mx_kvcache_compat", compat)
    monkeypatch.setenv("MXFLASHATTN_GRAPH_OFFICIAL_SPLIT", "1")
    assert _forward(mod) == "mx_kvcache"
    assert seen["official"] is vendor            # the compat wrapper can hand back
    assert fa.flash_attn_with_kvcache is vendor  # restored after the call
    assert native_decode.official_kvcache is None
    assert backend.get_dispatch_events() == [
        {"path": "vendor_direct", "operation": "official_split_mx", "fallback": "false"}]


def test_official_split_retries_vendor_after_invalid_argument(plugin, monkeypatch):
    """Mirrors the reference's test_official_split_retries_vendor_after_invalid_argument."""
    mod, fa = plugin
    calls = []

    def compat(*args, **kwargs):
        calls.append(1)
        raise RuntimeError("HIP error: invalid argument")

    monkeypatch.setattr(native_decode, "mx_kvcache_compat", compat)
    monkeypatch.setenv("MXFLASHATTN_GRAPH_OFFICIAL_SPLIT", "1")
    assert _forward(mod) == "vendor_kvcache"
    assert calls == [1]
    assert backend.get_dispatch_events() == [{
        "path": "vendor_direct",
        "operation": "official_split_invalid_argument_fallback",
        "fallback": "true",
        "fallback_reason": "official_split_invalid_argument",
    }]


def test_official_split_other_errors_propagate_and_restore(plugin, monkeypatch):
    mod, fa = plugin
    vendor = fa.flash_attn_with_kvcache

    def compat(*args, **kwargs):
        raise ValueError("shape")

    monkeypatch.setattr(native_decode, "mx_kvcache_compat", compat)
    monkeypatch.setenv("MXFLASHATTN_GRAPH_OFFICIAL_SPLIT", "1")
    with pytest.raises(ValueError, match="shape"):
        _forward(mod)
    assert fa.flash_attn_with_kvcache is vendor
    assert native_decode.official_kvcache is None
    assert backend.get_dispatch_events() == []

    # A module that had no such global gets none back (no None left behind).
    del fa.flash_attn_with_kvcache
    with pytest.raises(Exception):
        _forward(mod)
    assert "flash_attn_with_kvcache" not in fa.__dict__


def test_profiling_run_zero_fills_the_output(plugin):
    mod, _ = plugin
    out = torch.ones(3, 4)
    assert _forward(mod, metadata=None, output=out) is out
    assert not out.any()
    with pytest.raises(ValueError, match="output buffer for profiling"):
        _forward(mod, metadata=None, output=None)


def test_pure_split_encoders_and_default_fp8_go_to_vllm(plugin, monkeypatch):
    mod, _ = plugin
    monkeypatch.setattr(mod, "forward_decode",
                        lambda *a, **k: pytest.fail("must not reach the decode adapter"))
    monkeypatch.setenv("MXFLASHATTN_SPLIT_PURE", "1")
    assert _forward(mod) == "vendor_kvcache"
    monkeypatch.delenv("MXFLASHATTN_SPLIT_PURE")
    for attn_type in ("encoder", "encoder_only"):
        assert _forward(mod, mod.MXFlashAttnImpl(attn_type=attn_type)) == "vendor_kvcache"
    assert [e["operation"] for e in backend.get_dispatch_events()] == ["encoder", "encoder"]
    assert _forward(mod, mod.MXFlashAttnImpl(kv_cache_dtype="fp8")) == "vendor_kvcache"


@pytest.mark.parametrize("attr,value,reason", [
    ("alibi_slopes", torch.zeros(8), "alibi"),
    ("sliding_window", (127, 0), "window"),
    ("sliding_window", (0, 0), "window"),
    ("logits_soft_cap", 30.0, "softcap"),
    ("sinks", torch.zeros(8), "attention_sinks"),
])
def test_layer_options_the_kernel_lacks_run_vllms_forward(plugin, monkeypatch, attr, value,
                                                          reason):
    # The reference's forward decodes such layers without them.
    mod, _ = plugin
    monkeypatch.setattr(mod, "forward_decode",
                        lambda *a, **k: pytest.fail("must not reach the decode adapter"))
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (-1, -1), 0.0   # vLLM's defaults
    setattr(impl, attr, value)
    assert _forward(mod, impl) == "vendor_kvcache"
    assert backend.get_dispatch_events() == [
        {"path": "vendor_direct", "operation": "layer_option", "fallback": "true",
         "fallback_reason": reason}]


def test_quantised_output_goes_to_vllm(plugin, monkeypatch):
    mod, _ = plugin
    monkeypatch.setattr(mod, "forward_decode",
                        lambda *a, **k: pytest.fail("must not reach the decode adapter"))
    impl = mod.MXFlashAttnImpl()
    assert impl.forward(None, "q", "k", "v", "kv", "meta", "out", output_scale="s") == \
        "vendor_kvcache"
    assert backend.get_dispatch_events()[-1]["fallback_reason"] == "output_quantization"


def test_sliding_window_layers_decode_here_under_the_wider_contract(plugin, monkeypatch):
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: seen.append(k) or "decoded")
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (1023, 0), 0.0  # vLLM's form of a 1024 window
    assert _forward(mod, impl) == "decoded"
    assert seen[0]["window_left"] == 1023


def test_sink_layers_decode_here_under_the_wider_contract(plugin, monkeypatch):
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: seen.append(k) or "decoded")
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (127, 0), 0.0
    impl.sinks = torch.linspace(-1.0, 1.0, 8, dtype=torch.bfloat16)
    query = torch.zeros(4, 8, 64)
    assert impl.forward(None, query, None, None, "kv", "meta", "out") == "decoded"
    assert seen[0]["window_left"] == 127
    assert seen[0]["softcap"] == 0.0
    assert seen[0]["sinks"].dtype == torch.float32
    assert torch.equal(seen[0]["sinks"], impl.sinks.float())


def test_soft_capped_layers_decode_here_under_the_wider_contract(plugin, monkeypatch):
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: seen.append(k) or "decoded")
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (-1, -1), 50.0
    assert _forward(mod, impl) == "decoded"
    assert seen[0]["softcap"] == 50.0


def test_alibi_layers_decode_here_under_the_wider_contract(plugin, monkeypatch):
    # vLLM builds the slopes on the host; the kernel gets one device copy per layer.
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: seen.append(k) or "decoded")
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (-1, -1), 0.0
    impl.alibi_slopes = torch.pow(2.0, -torch.arange(1, 9, dtype=torch.float32))
    query = torch.zeros(4, 8, 64, device="meta")
    for _ in range(2):
        assert impl.forward(None, query, None, None, "kv", "meta", "out") == "decoded"
    assert seen[0]["alibi_slopes"].device.type == "meta"
    assert seen[0]["alibi_slopes"].shape == (8,)
    assert seen[1]["alibi_slopes"] is seen[0]["alibi_slopes"]  # copied once


@pytest.mark.parametrize("attr,value,reason", [
    ("alibi_slopes", torch.zeros(4, 8), "alibi"),      # per sequence: vLLM's
    ("sinks", torch.zeros(7), "attention_sinks"),
])
def test_per_head_vectors_of_another_shape_run_vllms_forward(plugin, monkeypatch, attr, value,
                                                             reason):
    mod, _ = plugin
    monkeypatch.setattr(mod, "forward_decode",
                        lambda *a, **k: pytest.fail("must not reach the decode adapter"))
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    impl = mod.MXFlashAttnImpl()
    impl.sliding_window, impl.logits_soft_cap = (-1, -1), 0.0
    setattr(impl, attr, value)
    assert impl.forward(None, torch.zeros(4, 8, 64), None, None, "kv", "meta", "out") == \
        "vendor_kvcache"
    assert backend.get_dispatch_events()[-1]["fallback_reason"] == reason


def test_layer_defaults_reach_the_adapter(plugin, monkeypatch):
    mod, _ = plugin
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: "decoded")
    impl = mod.MXFlashAttnImpl()
    impl.alibi_slopes, impl.sliding_window, impl.logits_soft_cap, impl.sinks = (
        None, (-1, -1), 0.0, None)
    assert _forward(mod, impl) == "decoded"


def test_decode_goes_through_the_adapter_with_layer_scales(plugin, monkeypatch):
    mod, _ = plugin
    seen = []

    def fake_forward_decode(query, kv_cache, metadata, output, **kwargs):
        seen.append(kwargs)
        return "decoded"

    monkeypatch.setattr(mod, "forward_decode", fake_forward_decode)
    layer = types.SimpleNamespace(_k_scale="ks", _v_scale="vs")
    assert _forward(mod, layer=layer) == "decoded"
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    assert _forward(mod, mod.MXFlashAttnImpl(kv_cache_dtype="fp8"), layer=layer) == "decoded"
    assert seen == [
        dict(softmax_scale=0.125, kv_cache_dtype="auto", k_scale="ks", v_scale="vs",
             window_left=-1, sinks=None, alibi_slopes=None, softcap=0.0),
        dict(softmax_scale=0.125, kv_cache_dtype="fp8", k_scale="ks", v_scale="vs",
             window_left=-1, sinks=None, alibi_slopes=None, softcap=0.0)]
    with pytest.raises(ValueError, match="output buffer"):
        _forward(mod, output=None)


def test_blocked_decode_hands_prefill_back_and_raises_otherwise(plugin, monkeypatch):
    mod, _ = plugin
    reason = {}

    def blocked(*args, **kwargs):
        raise DecoderAdapterBlocked(reason["r"])

    monkeypatch.setattr(mod, "forward_decode", blocked)
    reason["r"] = "only_single_token_decode_supported:max_query_len=7"
    assert _forward(mod) == "vendor_kvcache"
    reason["r"] = "cascade_attention_not_supported_by_adapter"
    with pytest.raises(DecoderAdapterBlocked, match="cascade"):
        _forward(mod)
    assert backend.get_dispatch_events() == [
        {"path": "vendor_prefill_or_blocked",
         "reason": "only_single_token_decode_supported:max_query_len=7"},
        {"path": "vendor_prefill_or_blocked",
         "reason": "cascade_attention_not_supported_by_adapter"}]


@pytest.mark.parametrize("kv_dtype", ["fp8_e5m2", "fp8_inc", "fp8_ds_mla"])
def test_cache_formats_the_kernels_lack_stay_with_vllm(plugin, monkeypatch, kv_dtype):
    mod, _ = plugin
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: pytest.fail("decode adapter"))
    monkeypatch.setattr(mod, "kv_cache_update", lambda *a: pytest.fail("HIP cache update"))
    impl = mod.MXFlashAttnImpl(kv_cache_dtype=kv_dtype)
    assert _forward(mod, impl) == "vendor_kvcache"
    assert impl.do_kv_cache_update(None, "k", "v", "cache", "slots") == "vendor_cache_update"


def test_named_sixteen_bit_caches_run_here(plugin, monkeypatch):
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "forward_decode", lambda *a, **k: seen.append(k) or "decoded")
    monkeypatch.setattr(mod, "kv_cache_update", lambda *a: seen.append(a))
    for kv_dtype in ("auto", "bfloat16", "float16", "half"):
        impl = mod.MXFlashAttnImpl(kv_cache_dtype=kv_dtype)
        assert _forward(mod, impl) == "decoded"
        impl.do_kv_cache_update(types.SimpleNamespace(), "k", "v", "cache", "slots")
    assert len(seen) == 8


def test_kv_cache_update_passes_the_cache_dtype_and_layer_scales(plugin, monkeypatch):
    mod, _ = plugin
    seen = []
    monkeypatch.setattr(mod, "kv_cache_update", lambda *a: seen.append(a))
    impl = mod.MXFlashAttnImpl(kv_cache_dtype="fp8")
    impl.do_kv_cache_update(types.SimpleNamespace(_k_scale=2.0, _v_scale=3.0), "k", "v",
                            "cache", "slots")
    assert seen == [("k", "v", "cache", "slots", "fp8", 2.0, 3.0)]


def test_plugin_import_needs_vllm():
    try:
        import vllm  # noqa: F401
    except ImportError:
        pass
    else:
        pytest.skip("vLLM is installed")
    assert PLUGIN not in sys.modules  # the stand-in of the other tests is gone
    with pytest.raises(ImportError):
        importlib.import_module(PLUGIN)
