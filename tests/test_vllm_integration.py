"""vLLM-side routing without vLLM (mirrors tests/test_vllm_bridge.py and
tests/test_vllm_official_split_fallback.py of the reference, for the parts that
do not need vLLM installed): shape guards, the compat wrapper's hand-back,
dispatch events and the backend registration result."""

import collections
import json

import pytest
import torch

import mxflashattn_amd.dispatch as dispatch
from mxflashattn_amd.integrations.vllm import backend, native_decode
from mxflashattn_amd.integrations.vllm.backend import attention_forward


def kv_kwargs(q_heads=16, kv_heads=4, head_dim=128, dtype=torch.float16, page=16):
    return {
        "k_cache": torch.empty(1, page, kv_heads, head_dim, dtype=dtype),
        "v_cache": torch.empty(1, page, kv_heads, head_dim, dtype=dtype),
        "block_table": torch.zeros(1, 1, dtype=torch.int32),
        "cache_seqlens": torch.ones(1, dtype=torch.int32),
    }


def test_dense_vllm_bridge_delegates_to_public_api(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    q = torch.randn(3, 2, 64)
    k = torch.randn(4, 1, 64)
    v = torch.randn_like(k)
    with pytest.warns(RuntimeWarning, match="native_backend_requires_accelerator_tensor"):
        output = attention_forward(q, k, v, causal=True, scale=0.125)
    assert output.shape == q.shape
    assert torch.isfinite(output).all()


@pytest.mark.parametrize("head_dim,q_heads,kv_heads", [(256, 16, 4), (128, 24, 8)])
def test_official_kvcache_compat_falls_back_to_vendor_for_unsupported_shapes(
        monkeypatch, head_dim, q_heads, kv_heads):
    calls = []
    expected = object()
    args = (torch.empty(1, 1, q_heads, head_dim),)
    kwargs = kv_kwargs(q_heads, kv_heads, head_dim, dtype=torch.float32)
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    monkeypatch.setattr(native_decode, "official_kvcache",
                        lambda *a, **k: calls.append((a, k)) or expected)
    monkeypatch.setattr(native_decode.api, "flash_attn_with_kvcache",
                        lambda *a, **k: pytest.fail("unsupported shape must not enter the MX API"))
    assert native_decode.mx_kvcache_compat(*args, **kwargs) is expected
    assert calls == [(args, kwargs)]


def test_compat_hands_calls_back_to_vllm_unchanged(monkeypatch):
    # The reference strips vLLM-only keywords (vllm_plugin.py:335-339) for its
    # vendor wheel; vLLM's own function takes them, so a declined call goes
    # back exactly as vLLM made it.
    seen = {}
    monkeypatch.setattr(native_decode, "official_kvcache",
                        lambda *a, **k: seen.update(k) or "vendor")
    kwargs = kv_kwargs()
    kwargs.update(s_aux=None, scheduler_metadata=None, fa_version=3, q_descale=None,
                  k_descale=None, v_descale=None, return_softmax_lse=False)
    expected = dict(kwargs)
    assert native_decode.mx_kvcache_compat(torch.empty(1, 1, 16, 128), **kwargs) == "vendor"
    assert seen.keys() == expected.keys()
    assert all(seen[k] is expected[k] for k in expected)


@pytest.mark.parametrize("extra,reason", [
    (dict(s_aux=torch.zeros(16)), "attention_sinks"),
    (dict(return_softmax_lse=True), "softmax_lse"),
])
def test_compat_never_takes_sinks_or_lse_requests(monkeypatch, extra, reason):
    """The kernel has no sinks and returns no LSE: such calls reach vLLM with
    those keywords intact (the reference drops them and computes without)."""
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    seen = {}
    monkeypatch.setattr(native_decode, "official_kvcache",
                        lambda *a, **k: seen.update(k) or "vendor")
    monkeypatch.setattr(native_decode, "try_native_decode",
                        lambda *a, **k: pytest.fail("must not reach the kernel"))
    backend.clear_dispatch_events(truncate_log=False)
    kwargs = kv_kwargs()
    kwargs.update(extra)
    assert native_decode.mx_kvcache_compat(q_of(), **kwargs) == "vendor"
    for k, v in extra.items():
        assert seen[k] is v
    assert backend.get_dispatch_events() == [
        {"path": "native_decode", "fallback": "true", "fallback_reason": f"guard:{reason}"}]


def test_wide_compat_takes_sinks_of_one_logit_per_query_head(monkeypatch):
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    seen = []
    monkeypatch.setattr(native_decode, "official_kvcache", lambda *a, **k: "vendor")
    monkeypatch.setattr(native_decode, "try_native_decode",
                        lambda args, kwargs, kd, vd, sinks=None: seen.append(sinks) or "native")
    good = torch.linspace(-1, 1, 16, dtype=torch.bfloat16)
    assert native_decode.mx_kvcache_compat(q_of(), s_aux=good, **kv_kwargs()) == "native"
    assert seen[0].dtype == torch.float32 and torch.equal(seen[0], good.float())
    # Not one value per query head: handed back with s_aux intact.
    assert native_decode.mx_kvcache_compat(q_of(), s_aux=torch.zeros(8), **kv_kwargs()) == \
        "vendor"
    assert len(seen) == 1


def test_compat_without_vllm_function_refuses_what_the_api_cannot_do(monkeypatch):
    monkeypatch.setattr(native_decode, "official_kvcache", None)
    with pytest.raises(NotImplementedError, match="s_aux"):
        native_decode.mx_kvcache_compat(q_of(), s_aux=torch.zeros(16), **kv_kwargs())
    with pytest.raises(NotImplementedError, match="return_softmax_lse"):
        native_decode.mx_kvcache_compat(q_of(), return_softmax_lse=True, **kv_kwargs())


def q_of(q_heads=16, head_dim=128, dtype=torch.float16, rank=4):
    return torch.empty((1, 1, q_heads, head_dim) if rank == 4 else (1, q_heads, head_dim),
                       dtype=dtype)


@pytest.mark.parametrize("case,reason", [
    (dict(q_heads=16, kv_heads=4, head_dim=256), "head_dim"),
    (dict(q_heads=24, kv_heads=8, head_dim=128), "gqa_ratio"),
    (dict(q_heads=16, kv_heads=16, head_dim=128), "gqa_ratio"),
    (dict(q_heads=64, kv_heads=4, head_dim=128), "gqa_ratio"),
    (dict(q_heads=16, kv_heads=4, head_dim=128, dtype=torch.float32), "dtype"),
    (dict(q_heads=16, kv_heads=4, head_dim=128, page=24), "page_size"),
    (dict(q_heads=16, kv_heads=4, head_dim=128), "device"),
])
def test_native_guard_hands_back_unsupported_calls(case, reason):
    dtype = case.get("dtype", torch.float16)
    q = q_of(case["q_heads"], case["head_dim"], dtype)
    kwargs = kv_kwargs(case["q_heads"], case["kv_heads"], case["head_dim"], dtype,
                       case.get("page", 16))
    got, picked = native_decode._guard((q,), kwargs)
    assert got == reason and picked == ()


@pytest.mark.parametrize("extra,reason", [
    (dict(alibi_slopes=torch.zeros(16)), "alibi"),
    (dict(window_size=(128, 0)), "window"),
    (dict(window_size=(0, 0)), "window"),     # keeps only the query's own key
    (dict(window_size=(0, -1)), "window"),
    (dict(window_size=5), "window"),
    (dict(window_size="wide"), "window"),
    (dict(softcap=30.0), "softcap"),
    (dict(block_table=None), "block_table_or_seqlens"),
    (dict(cache_seqlens=torch.ones(3, dtype=torch.int32)), "block_table_or_seqlens"),
])
def test_native_guard_option_checks(extra, reason):
    kwargs = kv_kwargs()
    kwargs.update(extra)
    assert native_decode._guard((q_of(),), kwargs)[0] == reason


def _guard_reason(window, causal, ql):
    kwargs = kv_kwargs()
    kwargs.update(window_size=window, causal=causal, softcap=0.0)
    q = torch.empty(1, ql, 16, 128, dtype=torch.float16)
    return native_decode._guard((q,), kwargs, native_decode.wide_contract())[0]


def test_native_guard_window_right_bound_matters_only_for_later_keys(monkeypatch):
    # The reference's contract: any window that masks something is handed back.
    # One query token, or causal masking, sees no key after itself: a right
    # bound of 0 masks nothing there. Several non-causal tokens would.
    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    for window, causal, ql, reason in (((-1, 0), False, 1, "device"),
                                       ((-1, 0), True, 3, "query_length"),
                                       ((-1, 0), False, 3, "window"),
                                       ((-1, -1), False, 1, "device"),
                                       (-1, False, 1, "device"),
                                       ((127, 0), True, 1, "window")):
        assert _guard_reason(window, causal, ql) == reason, (window, causal, ql)


def test_wide_guard_takes_soft_capping(monkeypatch):
    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    kwargs = dict(kv_kwargs(), softcap=30.0)
    assert native_decode._guard((q_of(),), kwargs)[0] == "softcap"
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    reason, picked = native_decode._guard((q_of(),), kwargs, True)
    assert reason == "device"   # every other guard passed on host tensors
    for bad in (-1.0, float("inf"), "x"):
        assert native_decode._guard((q_of(),), dict(kv_kwargs(), softcap=bad), True)[0] == \
            "softcap"


def test_wide_guard_takes_alibi_slopes_of_one_per_query_head(monkeypatch):
    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    slopes = torch.pow(2.0, -torch.arange(1, 17, dtype=torch.float64))
    kwargs = dict(kv_kwargs(), alibi_slopes=slopes)
    assert native_decode._guard((q_of(),), kwargs)[0] == "alibi"
    assert native_decode._guard((q_of(),), kwargs, True)[0] == "device"  # every other passed
    assert native_decode._sinks_for_kernel(slopes, q_of()).dtype == torch.float32
    for bad in (torch.zeros(1, 16), torch.zeros(15), [0.5] * 16):  # per sequence, short, list
        assert native_decode._guard((q_of(),), dict(kv_kwargs(), alibi_slopes=bad),
                                    True)[0] == "alibi"


def test_wide_guard_takes_sliding_windows(monkeypatch):
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    for window, causal, ql, reason in (((127, 0), True, 1, "device"),
                                       ((0, 0), False, 1, "device"),
                                       ((5, -1), False, 3, "device"),
                                       ((-1, 0), False, 3, "device"),   # right 0 = causal
                                       ((-1, 2), False, 3, "window"),   # no kernel bound
                                       ((4, 2), True, 3, "device"),
                                       ("wide", True, 1, "window")):
        assert _guard_reason(window, causal, ql) == reason, (window, causal, ql)
    assert native_decode.window_for_kernel((127, 0), False, 1) == (127, False)
    assert native_decode.window_for_kernel((-1, 0), False, 3) == (-1, True)
    assert native_decode.window_for_kernel((7, 0), False, 2) == (7, True)
    assert native_decode.window_for_kernel(None, True, 2) == (-1, True)
    assert native_decode.window_for_kernel((3, 5), False, 2) is None


def test_native_guard_accepts_no_window_and_rank3_queries():
    kwargs = kv_kwargs()
    kwargs["window_size"] = (-1, -1)
    # Host tensors reach the device check last: every shape check has passed.
    assert native_decode._guard((q_of(rank=3),), kwargs)[0] == "device"
    assert native_decode._guard((torch.empty(1, 2, 16, 128, dtype=torch.float16),),
                                kwargs)[0] == "query_length"


def test_native_decode_is_opt_in(monkeypatch):
    monkeypatch.delenv("MXFA_NATIVE_DECODE", raising=False)
    assert native_decode.try_native_decode((q_of(),), kv_kwargs()) is None


def test_guard_failures_are_recorded_as_fallback_events(monkeypatch):
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    backend.clear_dispatch_events(truncate_log=False)
    assert native_decode.try_native_decode((q_of(head_dim=256),),
                                           kv_kwargs(head_dim=256)) is None
    assert backend.get_dispatch_events() == [{
        "path": "native_decode", "fallback": "true", "fallback_reason": "guard:head_dim"}]


def test_dispatch_log_sampling(monkeypatch, tmp_path):
    log = tmp_path / "events.jsonl"
    monkeypatch.setenv("MXFLASHATTN_DISPATCH_LOG", str(log))
    monkeypatch.setenv("MXFLASHATTN_DISPATCH_SAMPLE", "3")
    backend.clear_dispatch_events()
    monkeypatch.setattr(backend, "_counter", 0)
    for i in range(7):
        backend.record_event({"path": "mi355x_split_decode", "i": str(i)})
    lines = [json.loads(x) for x in log.read_text().splitlines()]
    assert [x["i"] for x in lines] == ["0", "3", "6"]
    assert len(backend.get_dispatch_events()) == 7


def test_dispatch_event_buffer_keeps_the_most_recent(monkeypatch, tmp_path):
    # One event per layer per step: the in-memory buffer is bounded (oldest
    # dropped), while the log file, when set, keeps every line.
    assert backend.DISPATCH_EVENTS.maxlen == backend.DISPATCH_EVENTS_MAX == 65536
    log = tmp_path / "events.jsonl"
    monkeypatch.setenv("MXFLASHATTN_DISPATCH_LOG", str(log))
    monkeypatch.delenv("MXFLASHATTN_DISPATCH_SAMPLE", raising=False)
    monkeypatch.setattr(backend, "DISPATCH_EVENTS", collections.deque(maxlen=4))
    for i in range(10):
        backend.record_event({"path": "mi355x_split_decode", "i": str(i)})
    assert [e["i"] for e in backend.get_dispatch_events()] == ["6", "7", "8", "9"]
    assert len(log.read_text().splitlines()) == 10
    backend.clear_dispatch_events()
    assert backend.get_dispatch_events() == []


def test_plugin_import_log_names_the_dispatch_log(monkeypatch, tmp_path):
    monkeypatch.delenv("MXFLASHATTN_DISPATCH_LOG", raising=False)
    monkeypatch.setenv("MXFLASHATTN_PLUGIN_IMPORT_LOG", str(tmp_path / "run.plugin.log"))
    assert backend._log_path() == str(tmp_path / "run.dispatch.jsonl")


def test_registration_reports_missing_vllm():
    result = backend.register_vllm_v1_backend()
    try:
        import vllm  # noqa: F401
    except ImportError:
        assert result["registered"] == "false"
        assert result["reason"].startswith("vllm_v1_api_unavailable")


def test_reshape_and_cache_flash_cache_dtypes():
    # Other quantised formats are not supported.
    with pytest.raises(NotImplementedError, match="fp8_e5m2"):
        native_decode.reshape_and_cache_flash(None, None, None, None, torch.zeros(1), "fp8_e5m2")
    # Named 16-bit cache types are the plain copy (host tensors: refused at the device check).
    k16 = torch.zeros(2, 2, 64, dtype=torch.bfloat16)
    c16 = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16)
    for name in ("bfloat16", "float16", "half"):
        with pytest.raises(ValueError, match="GPU tensors"):
            native_decode.reshape_and_cache_flash(k16, k16, c16, c16,
                                                  torch.zeros(2, dtype=torch.int64), name)
    # "fp8" needs e4m3fn caches (or their uint8 codes).
    k = torch.zeros(2, 2, 64, dtype=torch.bfloat16)
    cache = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="uint8/e4m3fn"):
        native_decode.reshape_and_cache_flash(k, k, cache, cache, torch.zeros(2), "fp8")
    # uint8 caches are viewed as e4m3fn; host tensors are then refused.
    codes = torch.zeros(4, 16, 2, 64, dtype=torch.uint8)
    with pytest.raises(ValueError, match="GPU tensors"):
        native_decode.reshape_and_cache_flash(k, k, codes, codes, torch.zeros(2), "fp8")


def test_guard_wide_contract_opt_in(monkeypatch):
    """The reference's guards by default; MXFA_WIDE_CONTRACT=1 widens them to
    head dim 256, GQ 1..16 and fp8 caches with per-tensor descales."""
    def call(hq, hkv, hd, cache_dtype=torch.bfloat16, descale=None):
        q = torch.empty(4, 1, hq, hd, dtype=torch.bfloat16)
        cache = torch.empty(10, 16, hkv, hd, dtype=cache_dtype)
        kwargs = {"k_cache": cache, "v_cache": cache, "block_table": torch.zeros(4, 2),
                  "cache_seqlens": torch.ones(4)}
        wide = native_decode.wide_contract()
        return native_decode._guard((q,), kwargs, wide, (descale, descale))[0]

    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    assert call(16, 4, 256) == "head_dim"
    assert call(24, 8, 128) == "gqa_ratio"
    assert call(32, 8, 128, torch.float8_e4m3fn) == "dtype"
    monkeypatch.setenv("MXFA_WIDE_CONTRACT", "1")
    # Host tensors get as far as the device check: every shape guard passed.
    assert call(16, 4, 256) == "device"
    assert call(24, 8, 128) == "device"
    assert call(8, 8, 64) == "device"
    assert call(32, 8, 128, torch.float8_e4m3fn) == "device"
    scalar = torch.ones(1, dtype=torch.float32).expand(4, 8)
    assert call(32, 8, 128, torch.float8_e4m3fn, scalar) == "device"
    assert call(32, 8, 128, torch.float8_e4m3fn, torch.ones(4, 8)) == "descale_not_per_tensor"
    assert call(34, 2, 128) == "gqa_ratio"
    assert call(32, 8, 96) == "head_dim"

    def call_ql(ql, hq, hkv):
        q = torch.empty(4, ql, hq, 128, dtype=torch.bfloat16)
        cache = torch.empty(10, 16, hkv, 128, dtype=torch.bfloat16)
        kwargs = {"k_cache": cache, "v_cache": cache, "block_table": torch.zeros(4, 2),
                  "cache_seqlens": torch.ones(4), "causal": True}
        return native_decode._guard((q,), kwargs, native_decode.wide_contract())[0]

    assert call_ql(4, 32, 8) == "device"       # 4 tokens x GQ 4 = 16 columns
    assert call_ql(5, 32, 8) == "device"       # causal: two token chunks
    assert call_ql(16, 32, 8) == "device"      # 64 columns, four chunks
    assert call_ql(17, 32, 8) == "query_length"
    monkeypatch.delenv("MXFA_WIDE_CONTRACT")
    assert call_ql(2, 32, 8) == "query_length"  # the reference's guard


def test_vllm_compat_release_gate(tmp_path):
    """Mirrors tests/test_vllm_compat.py of the reference, plus local labels and the report."""
    from mxflashattn_amd.integrations.vllm import compat

    result = compat.classify_vllm("0.17.0")
    assert result.supported and result.status == "supported"
    assert compat.classify_vllm("0.17.1+rocm700").status == "supported"
    result = compat.classify_vllm("0.30.0")
    assert not result.supported and result.status == "probe_required"
    assert compat.classify_vllm(None).status == "not_installed"
    assert compat.classify_vllm("future-build").status == "unknown"
    assert compat.classify_vllm("7").status == "unknown"
    assert compat.classify_vllm("0.40.0").status == "unsupported"
    assert compat.classify_vllm("0.16.2").status == "unsupported"
    out = tmp_path / "r" / "vllm.json"
    report = compat.main(["--output", str(out)])
    assert json.loads(out.read_text()) == report
    assert report["status"] == compat.classify_vllm(compat.detect_vllm_version()).status


def _start_worker(tmp_path, env_extra, code, shadow=None):
    import os
    import pathlib
    import subprocess
    import sys

    root = pathlib.Path(__file__).resolve().parents[1]
    hook = root / "mxflashattn_amd" / "integrations" / "vllm" / "autoregister"
    env = {k: v for k, v in os.environ.items()
           if k not in ("MXFLASHATTN_AUTOREGISTER", "MXFLASHATTN_REGISTRATION_ERROR_LOG")}
    env["PYTHONPATH"] = os.pathsep.join([str(hook)] + ([str(shadow)] if shadow else []) +
                                        [str(root)])
    env.update(env_extra)
    return subprocess.run([sys.executable, "-c", code], env=env, cwd=tmp_path,
                          capture_output=True, text=True, timeout=120)


def test_autoregister_hook_runs_only_when_asked(tmp_path):
    """The sitecustomize hook (reference sitecustomize.py:8-17) in a fresh process."""
    probe = ("import sys; print('mxflashattn_amd.integrations.vllm.backend' in sys.modules, "
             "sys.modules['sitecustomize'].__file__)")
    off = _start_worker(tmp_path, {}, probe)
    assert off.returncode == 0, off.stderr
    assert off.stdout.split()[0] == "False" and "autoregister" in off.stdout
    on = _start_worker(tmp_path, {"MXFLASHATTN_AUTOREGISTER": "1"}, probe)
    assert on.returncode == 0, on.stderr
    assert on.stdout.split()[0] == "True"


def test_autoregister_hook_logs_failures_and_lets_the_worker_start(tmp_path):
    log = tmp_path / "reg.log"
    # A package that fails to import, ahead of the real one on the path, stands
    # for any failure inside registration.
    shadow = tmp_path / "shadow"
    (shadow / "mxflashattn_amd").mkdir(parents=True)
    (shadow / "mxflashattn_amd" / "__init__.py").write_text("raise RuntimeError('boom')\n")
    run = _start_worker(tmp_path, {"MXFLASHATTN_AUTOREGISTER": "1",
                                   "MXFLASHATTN_REGISTRATION_ERROR_LOG": str(log)},
                        "print('worker up')", shadow=shadow)
    assert run.returncode == 0, run.stderr
    assert run.stdout.strip() == "worker up"
    assert log.read_text() == "RuntimeError: boom\n"


def _picked_guard(monkeypatch):
    # Host tensors stop at the device check; pretend every guard passed.
    monkeypatch.setattr(native_decode, "_guard",
                        lambda args, kwargs, *a: (None, (args[0], kwargs["k_cache"],
                                                         kwargs["v_cache"],
                                                         kwargs["block_table"],
                                                         kwargs["cache_seqlens"], -1, False,
                                                         0.0, None)))
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    monkeypatch.setattr(native_decode.native, "default_num_splits", lambda *a: 4)


def test_native_decode_keeps_an_explicit_zero_scale(monkeypatch):
    _picked_guard(monkeypatch)
    seen = []
    monkeypatch.setattr(native_decode.native, "paged_decode_split",
                        lambda q, k, v, bt, sl, scale, **kw: seen.append(scale) or q)
    native_decode.try_native_decode((q_of(),), dict(kv_kwargs(), softmax_scale=0.0))
    native_decode.try_native_decode((q_of(),), kv_kwargs())
    assert seen == [0.0, 128 ** -0.5]


def test_native_decode_errors_hand_back_but_a_missing_build_raises(monkeypatch):
    _picked_guard(monkeypatch)
    backend.clear_dispatch_events(truncate_log=False)

    def unsupported(*a, **k):
        raise native_decode.native.UnsupportedConfig("page stride")

    monkeypatch.setattr(native_decode.native, "paged_decode_split", unsupported)
    assert native_decode.try_native_decode((q_of(),), kv_kwargs()) is None
    event = backend.get_dispatch_events()[-1]
    assert event["fallback"] == "true" and "page stride" in event["fallback_reason"]

    def missing(*a, **k):
        raise native_decode.native.NativeLibraryError("native library not built")

    monkeypatch.setattr(native_decode.native, "paged_decode_split", missing)
    with pytest.raises(native_decode.native.NativeLibraryError):
        native_decode.try_native_decode((q_of(),), kv_kwargs())
