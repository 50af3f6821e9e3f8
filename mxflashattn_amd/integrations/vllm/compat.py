"""Which vLLM releases the backend plugin's contract was validated against.

Mirrors ``integrations/vllm/compat.py:15-46`` of the reference: the plugin
(backend class path, ``do_kv_cache_update`` and ``forward`` signatures, the
decode metadata fields read by ``decoder_adapter``) follows vLLM 0.17's v1
attention-backend API. 0.30 changed that API and is reported as needing a probe
on the target environment; any other parsable release is unsupported. The
status strings are part of the interface (reports and dashboards key on them).

``python -m mxflashattn_amd.integrations.vllm.compat --output report.json``
writes the report for the current environment, as the reference's
``probe_compat.py:11-18`` does; nothing in vLLM is imported.
"""

from __future__ import annotations

import argparse
import importlib.metadata
import json
from dataclasses import asdict, dataclass
from pathlib import Path

SUPPORTED_RELEASE = (0, 17)
PROBE_RELEASE = (0, 30)


@dataclass(frozen=True)
class VllmCompatibility:
    installed_version: str | None
    status: str  # supported | probe_required | unsupported | unknown | not_installed
    reason: str
    supported: bool


def detect_vllm_version() -> str | None:
    """Installed vLLM distribution version from package metadata, or None."""
    try:
        return importlib.metadata.version("vllm")
    except importlib.metadata.PackageNotFoundError:
        return None


def _release(version: str) -> tuple[int, int] | None:
    # "0.17.0+rocm700" -> (0, 17); the local label after "+" is ignored.
    fields = version.split("+", 1)[0].split(".")
    if len(fields) < 2:
        return None
    try:
        return int(fields[0]), int(fields[1])
    except ValueError:
        return None


def classify_vllm(version: str | None) -> VllmCompatibility:
    if version is None:
        return VllmCompatibility(None, "not_installed", "vLLM is not installed", False)
    release = _release(version)
    if release is None:
        return VllmCompatibility(version, "unknown", "cannot parse vLLM version", False)
    if release == SUPPORTED_RELEASE:
        return VllmCompatibility(version, "supported", "v1.3 backend contract", True)
    if release == PROBE_RELEASE:
        return VllmCompatibility(
            version, "probe_required",
            "vLLM 0.30 API must be inspected and tested in the target environment", False)
    return VllmCompatibility(
        version, "unsupported",
        "no validated MXFlashAttn integration contract for this vLLM version", False)


def main(argv: list[str] | None = None) -> dict:
    parser = argparse.ArgumentParser(description=__doc__.split("\n", 1)[0])
    parser.add_argument("--output", type=Path, default=Path("artifacts/vllm-compatibility.json"))
    args = parser.parse_args(argv)
    report = asdict(classify_vllm(detect_vllm_version()))
    args.output.parent.mkdir(parents=True, exist_ok=True)
    text = json.dumps(report, indent=2) + "\n"
    args.output.write_text(text, encoding="utf-8")
    print(text, end="")
    return report


if __name__ == "__main__":
    main()
