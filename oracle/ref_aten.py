"""Loader of the reference's own ATen build in oracle/_ref/ (test infrastructure only).

``load()`` returns the module built by oracle/build_ref.py from the
reference's csrc/mxmac sources (functions flash_attn_with_kvcache,
flash_attn_func, flash_attn_varlen_func with the reference's signatures,
csrc/mxmac/attention_forward.cpp:104-116, paged_kv.cpp:53-126), or None when it has not been built.
Tests use it to pin the restatement in reference_port; bench.py times it as
the CPU baseline ("reference").
"""

from __future__ import annotations

import importlib.util
import sys

from .build_ref import MODULE, output_path


def load():
    path = output_path()
    if not path.exists():
        return None
    if MODULE in sys.modules:
        return sys.modules[MODULE]
    spec = importlib.util.spec_from_file_location(MODULE, path)
    module = importlib.util.module_from_spec(spec)
    import torch  # noqa: F401  (the module links torch's libraries)

    spec.loader.exec_module(module)
    sys.modules[MODULE] = module
    return module
