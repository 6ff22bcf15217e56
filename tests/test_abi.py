"""CPU checks of the C ABI: the library loads and exports every declared entry point."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

from nano_vllm_ascend_amd import _C

HEADER = Path(__file__).resolve().parents[1] / "include" / "nvamd.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(nvamd_\w+)\s*\(", text))


def test_header_and_binding_agree():
    assert declared_symbols() == set(_C.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = _C.load()
    for name in declared_symbols():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_host_only_entry_points():
    header = (Path(__file__).resolve().parents[1] / "include" / "nvamd.h").read_text()
    declared = int(re.search(r"#define NVAMD_ABI_VERSION (\d+)", header).group(1))
    assert _C.version() == declared
    small = _C.paged_decode_workspace_size(4, 16, 8, 512)
    big = _C.paged_decode_workspace_size(32, 16, 8, 4096)
    assert 0 < small < big
    assert _C.paged_decode_workspace_size(0, 16, 8, 512) == 0


def test_build_rejects_kernels_that_spill_to_scratch():
    """The build reads the compiler's kernel-resource-usage remarks and fails on any scratch use."""
    from nano_vllm_ascend_amd.build import scratch_by_kernel

    remarks = "\n".join([
        "a.hip:10:1: remark: Function Name: _Z3fooPf [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:10:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:10:1: remark:     ScratchSize [bytes/lane]: 116 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:20:1: remark: Function Name: _Z3barPf [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:20:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert scratch_by_kernel(remarks) == {"_Z3fooPf": 116, "_Z3barPf": 0}
    assert scratch_by_kernel("") == {}
