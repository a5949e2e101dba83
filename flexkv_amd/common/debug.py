"""Logger for the transfer path (role of flexkv/common/debug.py:9-58).

Level from FLEXKV_LOG_LEVEL (DEBUG, INFO, WARNING, ERROR, OFF; default INFO).
"""
from __future__ import annotations

import logging
import os
import sys


class FlexkvLogger:
    def __init__(self, name: str = "flexkv_amd") -> None:
        self._log = logging.getLogger(name)
        if not self._log.handlers:
            h = logging.StreamHandler(sys.stderr)
            h.setFormatter(logging.Formatter("[%(asctime)s] [%(name)s] [%(levelname)s] %(message)s"))
            self._log.addHandler(h)
        self._log.propagate = False
        self.set_level(os.environ.get("FLEXKV_LOG_LEVEL", "INFO"))

    def set_level(self, level: str) -> None:
        level = level.upper()
        if level == "OFF":
            self._log.setLevel(logging.CRITICAL + 10)
        else:
            self._log.setLevel(getattr(logging, level, logging.INFO))

    def enabled(self, level: str) -> bool:
        """Whether a message at `level` would be emitted (lets callers skip
        building messages nobody reads)."""
        return self._log.isEnabledFor(getattr(logging, level.upper(), logging.INFO))

    def debug(self, msg, *a) -> None:
        self._log.debug(msg, *a)

    def info(self, msg, *a) -> None:
        self._log.info(msg, *a)

    def warning(self, msg, *a) -> None:
        self._log.warning(msg, *a)

    def error(self, msg, *a) -> None:
        self._log.error(msg, *a)


flexkv_logger = FlexkvLogger()
