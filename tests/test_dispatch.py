"""Dispatch chain contract (mirrors the reference's tests/test_dispatch.py),
plus the MI355X decode backend's place at the head of the chain."""

from types import SimpleNamespace

import pytest
import torch

import mxflashattn_amd.dispatch as dispatch


@pytest.fixture(autouse=True)
def clear_provider_cache():
    dispatch._metax_flash_attn_module.cache_clear()
    yield
    dispatch._metax_flash_attn_module.cache_clear()


def test_flash_attn_provider_requires_metax_build(monkeypatch):
    fake_module = SimpleNamespace(flash_attn_func=lambda *args, **kwargs: None)
    monkeypatch.setenv("MXFLASHATTN_BACKEND", "auto")
    monkeypatch.setattr(dispatch.importlib, "import_module", lambda name: fake_module)
    monkeypatch.setattr(dispatch.importlib.metadata, "version", lambda name: "2.6.3")
    assert dispatch._flash_attn_function("flash_attn_func") is None


def test_flash_attn_provider_accepts_metax_build(monkeypatch):
    function = lambda *args, **kwargs: None  # noqa: E731
    fake_module = SimpleNamespace(flash_attn_func=function)
    versions = []
    monkeypatch.setenv("MXFLASHATTN_BACKEND", "auto")
    monkeypatch.setattr(dispatch.importlib, "import_module", lambda name: fake_module)
    monkeypatch.setattr(dispatch.importlib.metadata, "version",
                        lambda name: versions.append(name) or "2.6.3+metax3.5.3.9torch2.8")
    assert dispatch._flash_attn_function("flash_attn_func") is function
    assert dispatch._flash_attn_function("flash_attn_func") is function
    assert versions == ["flash-attn"]


def test_aten_override_skips_external_flash_attn(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_BACKEND", "aten")
    monkeypatch.setattr(
        dispatch.importlib, "import_module",
        lambda name: (_ for _ in ()).throw(AssertionError("must not import flash_attn")))
    assert dispatch._flash_attn_function("flash_attn_func") is None


def test_zero_scale_uses_aten_extension_even_when_metax_provider_exists(monkeypatch):
    calls = []
    provider = lambda *args, **kwargs: pytest.fail("MetaX provider must not receive zero scale")  # noqa: E731
    extension = SimpleNamespace(
        is_available=lambda: True,
        flash_attn_func=lambda *args: calls.append(args) or torch.tensor([1]),
    )
    tensor = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.float16)
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: provider)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: extension)
    result = dispatch.dispatch("flash_attn_func", tensor, (tensor,),
                               lambda: pytest.fail("fallback must not run"),
                               native_args=(tensor,), native_kwargs={"softmax_scale": 0.0})
    assert result.item() == 1
    assert calls == [(tensor,)]
    assert dispatch.get_last_dispatch_info().backend == "mxmac_aten_correctness"


def test_zero_scale_requires_aten_extension_if_metax_provider_is_present(monkeypatch):
    tensor = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.float16)
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: lambda *args: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    assert dispatch.native_unavailable_reason(tensor, "flash_attn_func", require_aten=True) == (
        "zero_softmax_scale_requires_aten_extension")


def test_qualifying_decode_route_runs_first_and_is_recorded(monkeypatch):
    monkeypatch.setattr(dispatch, "_flash_attn_function",
                        lambda operation: pytest.fail("vendor must not be consulted"))
    tensor = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.bfloat16)
    expected = object()
    route = dispatch.DecodeRoute(None, lambda: expected)
    result = dispatch.dispatch("flash_attn_with_kvcache", tensor, (), lambda: pytest.fail("no"),
                               native_args=(), native_kwargs={"softmax_scale": 0.0},
                               decode_route=route)
    assert result is expected
    info = dispatch.get_last_dispatch_info()
    assert info == dispatch.DispatchInfo("mi355x_split_decode", "flash_attn_with_kvcache", None)


def test_failures_of_a_qualifying_decode_route_propagate(monkeypatch):
    """No silent fallback: a call the HIP path takes either runs there or raises."""
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    tensor = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.bfloat16)

    def broken():
        raise RuntimeError("mxfa_split_decode_launch failed (-4)")

    with pytest.raises(RuntimeError, match="-4"):
        dispatch.dispatch("flash_attn_with_kvcache", tensor, (), lambda: pytest.fail("fallback"),
                          native_args=(), native_kwargs={},
                          decode_route=dispatch.DecodeRoute(None, broken))
    assert dispatch.get_last_dispatch_info() is None


def test_declined_decode_route_reason_joins_the_chain(monkeypatch):
    monkeypatch.delenv("MXFLASHATTN_ALLOW_FALLBACK", raising=False)
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    tensor = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.bfloat16)
    with pytest.raises(dispatch.BackendUnavailableError,
                       match="mi355x_split_decode:head_dim_256"):
        dispatch.dispatch("flash_attn_with_kvcache", tensor, (), lambda: None,
                          native_args=(), native_kwargs={},
                          decode_route=dispatch.DecodeRoute("head_dim_256_not_in_(64, 128)"))


def test_dispatch_info_is_thread_local():
    import threading

    dispatch._record(dispatch.DispatchInfo("reference", "flash_attn_func", "x"))
    seen = []
    thread = threading.Thread(target=lambda: seen.append(dispatch.get_last_dispatch_info()))
    thread.start()
    thread.join()
    assert seen == [None]
    assert dispatch.get_last_dispatch_info().backend == "reference"
