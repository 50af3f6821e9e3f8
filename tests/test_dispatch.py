"""The backend chain of mxflashattn_amd.dispatch, driven through a fake world.

A ``World`` fixture decides what the chain can see (a vendor flash_attn
function or none, an ATen extension or none, the fallback switch) and records
what each backend received. The chain's order, its recorded DispatchInfo and
the reason strings callers parse (mxflashattn/dispatch.py) are checked table
by table; the MI355X route at the head of the chain has its own cases.
"""

from __future__ import annotations

import threading
from types import SimpleNamespace

import pytest
import torch

import mxflashattn_amd.dispatch as dispatch

CUDA_F16 = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.float16)
CUDA_F32 = SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=torch.float32)
HOST_F16 = SimpleNamespace(device=SimpleNamespace(type="cpu"), dtype=torch.float16)


class World:
    """What the chain sees, and a log of which backend ran with what."""

    def __init__(self, monkeypatch):
        self.mp = monkeypatch
        self.log: list[tuple[str, object]] = []
        self.vendor = None
        self.extension = None
        monkeypatch.setattr(dispatch, "_flash_attn_function", lambda op: self.vendor)
        monkeypatch.setattr(dispatch, "_native_extension", lambda: self.extension)
        monkeypatch.delenv("MXFLASHATTN_ALLOW_FALLBACK", raising=False)

    def with_vendor(self, fails: bool = False):
        def vendor(*args, **kwargs):
            self.log.append(("vendor", kwargs))
            if fails:
                raise RuntimeError("vendor kernel refused the shape")
            return "vendor-result"
        self.vendor = vendor
        return self

    def with_extension(self, available: bool = True, implements: bool = True):
        ext = SimpleNamespace(is_available=lambda: available)
        if implements:
            ext.flash_attn_func = lambda *args: self.log.append(("aten", args)) or "aten-result"
        self.extension = ext
        return self

    def allow_fallback(self):
        self.mp.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
        return self

    def call(self, tensor=CUDA_F16, scale=None, route=None):
        return dispatch.dispatch(
            "flash_attn_func", tensor, ("ext-arg",),
            lambda: self.log.append(("reference", None)) or "reference-result",
            native_args=(), native_kwargs={"softmax_scale": scale}, decode_route=route)


@pytest.fixture
def world(monkeypatch):
    dispatch._metax_flash_attn_module.cache_clear()
    yield World(monkeypatch)
    dispatch._metax_flash_attn_module.cache_clear()


@pytest.mark.parametrize("setup,scale,backend,result", [
    (lambda w: w.with_vendor(), None, "vendor_direct", "vendor-result"),
    (lambda w: w.with_vendor().with_extension(), 0.5, "vendor_direct", "vendor-result"),
    (lambda w: w.with_extension(), None, "mxmac_aten_correctness", "aten-result"),
    # An explicit zero scale skips the vendor, which would read it as "default".
    (lambda w: w.with_vendor().with_extension(), 0.0, "mxmac_aten_correctness", "aten-result"),
    (lambda w: w.with_vendor(fails=True).with_extension(), None, "mxmac_aten_correctness",
     "aten-result"),
    (lambda w: w.allow_fallback(), None, "reference", "reference-result"),
    (lambda w: w.with_extension(available=False).allow_fallback(), None, "reference",
     "reference-result"),
])
def test_first_backend_that_serves_the_call_wins(world, setup, scale, backend, result):
    setup(world)
    with pytest.warns(RuntimeWarning) if backend == "reference" else _no_warning():
        assert world.call(scale=scale) == result
    assert dispatch.get_last_dispatch_info().backend == backend
    assert [name for name, _ in world.log][-1] == backend.split("_")[0].replace("mxmac", "aten")


class _no_warning:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


@pytest.mark.parametrize("setup,tensor,scale,reason", [
    (lambda w: w, CUDA_F16, None, "native_extension_not_built_or_not_importable"),
    (lambda w: w, HOST_F16, None, "native_backend_requires_accelerator_tensor"),
    (lambda w: w, CUDA_F32, None, "native_backend_supports_only_float16_and_bfloat16"),
    (lambda w: w.with_vendor(), CUDA_F16, 0.0, "zero_softmax_scale_requires_aten_extension"),
    (lambda w: w.with_extension(available=False), CUDA_F16, None,
     "native_extension_reports_unavailable_runtime"),
    (lambda w: w.with_extension(implements=False), CUDA_F16, None,
     "native_extension_does_not_implement_flash_attn_func"),
])
def test_refusal_names_the_reason_and_the_fallback_switch(world, setup, tensor, scale, reason):
    setup(world)
    with pytest.raises(dispatch.BackendUnavailableError) as info:
        world.call(tensor=tensor, scale=scale)
    assert reason in str(info.value)
    assert "MXFLASHATTN_ALLOW_FALLBACK=1" in str(info.value)
    assert dispatch.get_last_dispatch_info() is None


def test_vendor_failure_is_recorded_on_the_fallback(world):
    world.with_vendor(fails=True).allow_fallback()
    with pytest.warns(RuntimeWarning, match="vendor_call_failed:RuntimeError"):
        world.call()
    info = dispatch.get_last_dispatch_info()
    assert info.backend == "reference"
    assert info.fallback_reason.startswith("vendor_call_failed:RuntimeError:vendor kernel")


def test_mi355x_route_heads_the_chain(world):
    world.with_vendor().with_extension()
    route = dispatch.DecodeRoute(None, lambda: "hip-result")
    assert world.call(route=route) == "hip-result"
    assert world.log == []  # nothing else was consulted
    assert dispatch.get_last_dispatch_info() == dispatch.DispatchInfo(
        "mi355x_split_decode", "flash_attn_func", None)


def test_a_failing_mi355x_route_raises_instead_of_falling_back(world):
    world.with_vendor().allow_fallback()

    def launch():
        raise RuntimeError("mxfa_split_decode_launch failed (-4): kernel launch failed")

    with pytest.raises(RuntimeError, match=r"\(-4\)"):
        world.call(route=dispatch.DecodeRoute(None, launch))
    assert world.log == [] and dispatch.get_last_dispatch_info() is None


def test_a_declined_mi355x_route_adds_its_reason(world):
    world.with_extension().allow_fallback()
    world.call(route=dispatch.DecodeRoute("page_size_12_not_a_power_of_two_up_to_4096"))
    assert dispatch.get_last_dispatch_info().backend == "mxmac_aten_correctness"
    world.extension = None
    with pytest.warns(RuntimeWarning):
        world.call(route=dispatch.DecodeRoute("gqa_ratio_34/2_not_in_1..16"))
    reason = dispatch.get_last_dispatch_info().fallback_reason
    assert "mi355x_split_decode:gqa_ratio_34/2_not_in_1..16" in reason.split(";")


@pytest.mark.parametrize("version,accepted", [
    ("2.6.3", False),
    ("2.6.3+rocm6.4", False),
    ("2.6.3+metax3.5.3.9torch2.8", True),
    ("2.7.0+MetaX", True),
])
def test_only_a_metax_flash_attn_build_is_a_vendor(monkeypatch, version, accepted):
    fn = object()
    monkeypatch.setenv("MXFLASHATTN_BACKEND", "auto")
    monkeypatch.setattr(dispatch.importlib, "import_module",
                        lambda name: SimpleNamespace(flash_attn_func=lambda: fn))
    lookups = []
    monkeypatch.setattr(dispatch.importlib.metadata, "version",
                        lambda name: lookups.append(name) or version)
    dispatch._metax_flash_attn_module.cache_clear()
    try:
        first = dispatch._flash_attn_function("flash_attn_func")
        second = dispatch._flash_attn_function("flash_attn_func")
    finally:
        dispatch._metax_flash_attn_module.cache_clear()
    assert (first is not None) == accepted and first is second
    assert lookups == ["flash-attn"]  # probed once, then cached


def test_backend_aten_never_imports_flash_attn(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_BACKEND", "ATen ")

    def refuse(name):
        raise AssertionError(f"imported {name}")

    monkeypatch.setattr(dispatch.importlib, "import_module", refuse)
    assert dispatch._flash_attn_function("flash_attn_with_kvcache") is None


def test_dispatch_info_belongs_to_the_calling_thread(world):
    world.with_extension()
    world.call()
    seen = {}

    def other():
        seen["before"] = dispatch.get_last_dispatch_info()
        dispatch._record(dispatch.DispatchInfo("reference", "flash_attn_varlen_func", "x"))
        seen["after"] = dispatch.get_last_dispatch_info()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] is None and seen["after"].operation == "flash_attn_varlen_func"
    assert dispatch.get_last_dispatch_info().backend == "mxmac_aten_correctness"
