"""The persistent step's abort-word handling on the host (csrc/step_status.hpp), on the CPU.

An aborted persistent launch (a grid-barrier wait past its deadline) leaves invalid hidden states and
cache rows; every entry point that consumes or extends step results (cached steps, get_logits,
get_confidence, the unmask entry points) takes the abort word first and fails once instead of returning
results of the aborted launch, and the launching call itself checks by default whenever the persistent
path is on.  The helper is host code, so it is compiled with g++ and run here."""

from __future__ import annotations

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not available")
def test_step_abort_word_handling(tmp_path):
    exe = tmp_path / "step_status_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(ROOT / "fast-dllm-relax_amd" / "csrc"),
                    str(ROOT / "tests" / "step_status_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr


def test_entry_points_take_the_abort_word():
    """Every entry point that returns or extends step results takes the word before launching anything."""
    src = (ROOT / "fast-dllm-relax_amd" / "csrc" / "capi.hip").read_text()
    for fn in ("int cached_step(", "int fdllm_get_logits(", "int fdllm_get_confidence(",
               "int fdllm_get_confidence_unmask(", "int fdllm_unmask("):
        start = src.index(fn)
        body = src[start:src.index("\n}\n", start)]
        first_launch = min((body.find(k) for k in ("launch_", "run_lm_head", "run_layers", "try_step") if k in body),
                           default=len(body))
        assert "pending_step_abort(c)" in body[:first_launch], fn
