"""Module-global configuration with snapshot/restore (kernel_gen/core/config.py:95-349):
the current target and the dump directory for generated sources."""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

_TARGET: str | None = None
_DUMP_DIR: Path | None = None


@dataclass(frozen=True)
class ConfigSnapshot:
    target: str | None
    dump_dir: Path | None


def set_target(target: str | None) -> None:
    global _TARGET
    _TARGET = target


def get_target() -> str | None:
    return _TARGET


def set_dump_dir(path: str | Path | None) -> None:
    global _DUMP_DIR
    _DUMP_DIR = None if path is None else Path(path)


def get_dump_dir() -> Path | None:
    return _DUMP_DIR


def snapshot_config() -> ConfigSnapshot:
    return ConfigSnapshot(_TARGET, _DUMP_DIR)


def restore_config(snapshot: ConfigSnapshot) -> None:
    global _TARGET, _DUMP_DIR
    _TARGET, _DUMP_DIR = snapshot.target, snapshot.dump_dir
