"""The group-wait fault word on the host (csrc/wait_status.hpp), on the CPU.

A launch whose workgroups wait on each other (the down projection's k splits and the decode attention's
key splits reduced inside their own launch) bounds every wait; a wait that times out sets a fault word
and that launch's results are invalid.  Every entry point that consumes or extends step results (cached
steps, get_logits, get_confidence, the unmask entry points) takes the word first and fails once instead
of returning results computed after the faulted launch, and the in-launch reductions stay off for the
rest of the context's life.  The helper is host code, so it is compiled with g++ and run here."""

from __future__ import annotations

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not available")
def test_wait_fault_word_handling(tmp_path):
    exe = tmp_path / "wait_status_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(ROOT / "fast-dllm-relax_amd" / "csrc"),
                    str(ROOT / "tests" / "wait_status_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr


def test_entry_points_take_the_fault_word():
    """Every entry point that returns or extends step results takes the word before launching anything."""
    src = (ROOT / "fast-dllm-relax_amd" / "csrc" / "capi.hip").read_text()
    for fn in ("int cached_step(", "int cached_step_batch(", "int fdllm_forward_hidden(", "int fdllm_build_prefix_cache(", "int fdllm_build_prefix_cache_seq(", "int fdllm_get_logits(", "int fdllm_get_confidence(",
               "int fdllm_get_confidence_unmask(", "int fdllm_unmask("):
        start = src.index(fn)
        body = src[start:src.index("\n}\n", start)]
        first_launch = min((body.find(k) for k in ("launch_", "run_lm_head", "run_layers") if k in body),
                           default=len(body))
        assert "pending_wait_fault(c)" in body[:first_launch], fn


def test_group_waits_planned_only_for_resident_grids():
    """The place that plans an in-launch reduction checks the grid against the compute units."""
    src = (ROOT / "fast-dllm-relax_amd" / "csrc" / "capi.hip").read_text()
    assert src.count("group_waits_fit(c->group_waits, c->wait_fault,") == 1
