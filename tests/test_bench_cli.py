"""bench.py's command line without a GPU: more than one GPU is refused with
exit status 2 and a message, before anything touches a device."""

from __future__ import annotations

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused(capsys, monkeypatch):
    monkeypatch.delenv("WORLD_SIZE", raising=False)
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err


def test_a_distributed_launch_is_refused(capsys, monkeypatch):
    monkeypatch.setenv("WORLD_SIZE", "2")
    assert bench.main([]) == 2
    assert "WORLD_SIZE 2" in capsys.readouterr().err
