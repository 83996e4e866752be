"""JSON persistence for benchmark results and calibrated peaks.

Same contract as ``src/tklab/harness/jsonio.py``: ``read_json_object`` returns a
top-level JSON object (anything else is a ``ValueError``) and ``write_json_atomic``
replaces the destination in one rename, so a reader never sees a half-written file.
"""

from __future__ import annotations

import json
import os
import tempfile
from pathlib import Path
from typing import Any

JsonObject = dict[str, Any]


def read_json_object(path: Path) -> JsonObject:
    """Load ``path`` and require a top-level JSON object (reference ``jsonio.py:16-34``).

    Raises:
        ValueError: If the file is not valid JSON or its top level is not an object.
    """
    try:
        payload = json.loads(Path(path).read_text(encoding="utf-8"))
    except json.JSONDecodeError as error:
        raise ValueError(f"{path}: invalid JSON: {error}") from error
    if not isinstance(payload, dict):
        raise ValueError(f"{path}: expected a top-level JSON object")
    return payload


def write_json_atomic(path: Path, payload: JsonObject) -> None:
    """Write ``payload`` to ``path`` through a temporary file in the same directory
    and one ``os.replace`` (reference ``jsonio.py:37-69``)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=f".{path.name}.", suffix=".tmp", dir=path.parent)
    try:
        with os.fdopen(fd, "w", encoding="utf-8") as handle:
            json.dump(payload, handle, indent=2, sort_keys=True)
            handle.write("\n")
            handle.flush()
            os.fsync(handle.fileno())
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise
