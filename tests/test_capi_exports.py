"""The C ABI library loads and exports every entry point include/fdllm.h declares (no GPU calls)."""

import ctypes
import re

from conftest import ROOT

import fast_dllm_relax_amd._lib as lib


def _declared():
    text = (ROOT / "include" / "fdllm.h").read_text()
    return sorted(set(re.findall(r"\b(fdllm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_nine_entry_points():
    names = _declared()
    for fn in ("embed", "forward_hidden", "get_logits", "build_prefix_cache", "forward_cached",
               "forward_block_partial_rp0", "forward_block_partial_rp8", "forward_block_partial_rp16",
               "forward_block_partial_rp24"):
        assert f"fdllm_{fn}" in names


def test_library_exports_every_declared_symbol():
    so = lib.load()
    for name in _declared():
        assert hasattr(so, name), name
    assert sorted(lib.EXPORTS) == _declared()


def test_library_has_gfx950_code_object():
    data = lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data


def test_last_error_starts_empty():
    assert lib.load().fdllm_last_error() in (b"", None) or isinstance(lib.load().fdllm_last_error(), bytes)


def test_config_struct_layout_matches_header():
    # 13 four-byte fields, in header order
    assert ctypes.sizeof(lib.FdllmConfig) == 13 * 4
    assert [f[0] for f in lib.FdllmConfig._fields_][-2:] == ["dtype", "max_rows"]


def test_no_kernel_uses_scratch_memory():
    """The build keeps the compiler's per-kernel resource report beside the library: no kernel may spill
    to scratch (a private copy of a kernel-argument struct, or spilled registers, costs every wave
    global-memory round trips on the decode step's critical path)."""
    import pytest

    report = lib.LIB_PATH.parent / "kernel_resources.txt"
    if not report.exists():
        pytest.skip("no resource report (library built without the Makefile)")
    kernels, current = {}, None
    for line in report.read_text().splitlines():
        line = line.strip()
        if line.startswith("Function Name:"):
            current = line.split(":", 1)[1].strip()
        elif line.startswith("ScratchSize") and current is not None:
            kernels[current] = int(line.rsplit(":", 1)[1])
    assert kernels, "empty resource report"
    assert {k: v for k, v in kernels.items() if v} == {}
