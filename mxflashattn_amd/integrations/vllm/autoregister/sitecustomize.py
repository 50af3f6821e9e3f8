"""Worker-side registration of the MI355X backend in vLLM processes.

vLLM starts its workers as fresh Python processes, so a registration made in
the launching process does not reach them. Put this directory on PYTHONPATH
(with the directory holding ``mxflashattn_amd``) and set
MXFLASHATTN_AUTOREGISTER=1; Python then imports this module at start-up in
every process, and the hook calls ``register_vllm_v1_backend``. Without the
variable it does nothing. Failures never stop the worker: their type and
message are appended to the file named by MXFLASHATTN_REGISTRATION_ERROR_LOG,
if set. Behaves as the reference's ``sitecustomize.py:8-17``.
"""

import os

if os.getenv("MXFLASHATTN_AUTOREGISTER") == "1":
    try:
        from mxflashattn_amd.integrations.vllm.backend import register_vllm_v1_backend

        register_vllm_v1_backend()
    except Exception as exc:  # the worker must start whatever happens here
        _log = os.getenv("MXFLASHATTN_REGISTRATION_ERROR_LOG")
        if _log:
            with open(_log, "a", encoding="utf-8") as stream:
                stream.write(f"{type(exc).__name__}: {exc}\n")
