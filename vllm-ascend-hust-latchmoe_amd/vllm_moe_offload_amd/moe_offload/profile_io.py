"""Append-only JSONL writer for the runtime's profile events.

One line per event (keys sorted), written with a single unbuffered append
under a process-wide lock, so lines from several threads never interleave and
nothing is lost when the process ends without a flush.  One descriptor per
path stays open until exit.

Reference: moe_offload/profile_io.py:33-106 (append_jsonl and its flush and
close entry points); runtime.py:2900-2926 (which path the events go to).
"""

from __future__ import annotations

import atexit
import json
import os
from pathlib import Path
from threading import Lock

# environment names that point the runtime's events at a JSONL file, first hit wins
PROFILE_PATH_ENVS = (
    "VLLM_ASCEND_MOE_GMM_PROFILE_PATH",
    "VLLM_ASCEND_MOE_OFFLOAD_PROFILE_PATH",
    "VLLM_MOE_OFFLOAD_PROFILE_PATH",
)


def profile_path_from_env(configured: str = "") -> str:
    if configured:
        return str(configured)
    for name in PROFILE_PATH_ENVS:
        v = os.environ.get(name, "").strip()
        if v:
            return v
    return ""


class _AppendWriter:
    def __init__(self) -> None:
        self._lock = Lock()
        self._fds: dict[str, int] = {}

    def append(self, path, entry: dict) -> None:
        key = str(path)
        if not key:
            return
        data = (json.dumps(entry, sort_keys=True, default=_jsonable) + "\n").encode("utf-8")
        with self._lock:
            fd = self._fds.get(key)
            if fd is None:
                Path(key).parent.mkdir(parents=True, exist_ok=True)
                fd = os.open(key, os.O_WRONLY | os.O_CREAT | os.O_APPEND, 0o644)
                self._fds[key] = fd
            view = memoryview(data)
            while view:
                view = view[os.write(fd, view):]

    def close_all(self) -> None:
        with self._lock:
            fds, self._fds = list(self._fds.values()), {}
        for fd in fds:
            try:
                os.close(fd)
            except OSError:
                pass


def _jsonable(v):
    if hasattr(v, "to_jsonable"):
        return v.to_jsonable()
    if isinstance(v, (set, frozenset, tuple)):
        return list(v)
    return str(v)


_WRITER = _AppendWriter()
atexit.register(_WRITER.close_all)


def append_jsonl(path, entry: dict) -> None:
    _WRITER.append(path, entry)


def flush_profile_writes() -> None:
    """Lines are written unbuffered; nothing is held back."""


def close_profile_writes() -> None:
    _WRITER.close_all()
