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


# Argument checks run on the host before any HIP call, so they are testable without a GPU.  The
# addresses below are fake 16-byte-aligned device addresses that no failing call dereferences.
EINVAL, EUNSUPPORTED, EWORKSPACE, ETOOLARGE = -1, -2, -3, -4
A = 0x10000  # aligned stand-in address


def _fused(lib, **over):
    args = dict(out=A, out_stride=2048, q=A, q_stride=4096, k=A, k_stride=4096, v=A, v_stride=4096, qw=A, kw=A,
                positions=A, cos_sin=A, max_positions=4096, eps=1e-6, k_cache=A, v_cache=A, num_blocks=64,
                block_size=128, slots=A, bt=A, bt_stride=8, bt_width=8, ctx=A, batch=4, hq=16, hkv=8, d=128,
                scale=128 ** -0.5, max_ctx=1024, ws=A, ws_bytes=1 << 24, stream=None)
    args.update(over)
    return lib.nvamd_paged_decode_fused(*args.values())


def test_fused_decode_step_argument_errors():
    lib = _C.load()
    assert _fused(lib, batch=0) == 0                       # nothing to do
    assert _fused(lib, d=64) == EUNSUPPORTED               # head_dim must be 128
    assert _fused(lib, block_size=8) == EUNSUPPORTED       # block_size >= 16
    assert _fused(lib, hq=12) == EINVAL                    # Hq not a multiple of Hkv
    assert _fused(lib, k=A + 2) == EINVAL                  # misaligned new-token rows
    assert _fused(lib, k_stride=8 * 128 - 8) == EINVAL     # rows shorter than Hkv * D
    assert _fused(lib, cos_sin=A + 4) == EINVAL            # the rope table is read 16 bytes at a time
    assert _fused(lib, positions=0) == EINVAL
    assert _fused(lib, slots=0) == EINVAL
    assert _fused(lib, max_positions=0) == EINVAL
    assert _fused(lib, ws_bytes=16) == EWORKSPACE


def test_skinny_linear_argument_errors():
    lib = _C.load()

    def call(**over):
        args = dict(x=A, x_stride=1024, x_ssq=None, nw=None, eps=1e-6, w=A, y=A, y_stride=4096, y_ssq=None, epi=0,
                    flags=0, m=32, n=4096, k=1024, ws=None, ws_bytes=0, stream=None)
        args.update(over)
        return lib.nvamd_skinny_linear(*args.values())

    assert call(m=0) == 0
    assert call(m=129) == EUNSUPPORTED                     # at most 128 rows
    assert call(flags=4) == EINVAL                         # unknown flag
    assert call(x_stride=1000) == EINVAL                   # row-major x rows shorter than k
    assert call(w=A + 8) == EINVAL                         # the tiled weight is read 16 bytes at a time
    assert call(epi=2, y_ssq=None) == EINVAL               # the residual epilogue writes sums of squares


def test_paged_prefill_rejects_small_blocks():
    lib = _C.load()
    common = dict(out=A, out_stride=2048, q=A, q_stride=2048, k_cache=A, v_cache=A, num_blocks=64)
    tail = dict(bt=A, bt_stride=8, bt_width=8, cu=A, kv=A, n_seqs=2, max_q=64, hq=16, hkv=8, d=128,
                scale=128 ** -0.5, stream=None)
    for bs, want in ((8, EUNSUPPORTED), (12, EUNSUPPORTED)):
        assert lib.nvamd_paged_prefill(*common.values(), bs, *tail.values()) == want


def test_noalloc_decode_size_limit_is_checked_on_the_host():
    """The allocation-free decode refuses a call whose workspace would exceed the static scratch
    before it touches the device (fake addresses, no GPU needed)."""
    lib = _C.load()
    header = HEADER.read_text()
    assert "#define NVAMD_DECODE_SCRATCH_BYTES (64u * 1024u * 1024u)" in header
    assert _C.DECODE_SCRATCH_BYTES == 64 * 1024 * 1024
    args = [A, 2048, A, 2048, A, A, 64, 128, A, 8, 8, A, 4, 16, 8, 128, 128 ** -0.5]
    assert lib.nvamd_paged_decode_noalloc(*args, 2_621_440, None) == ETOOLARGE
    assert lib.nvamd_paged_decode_noalloc(*args[:12], 0, *args[13:], 1024, None) == 0  # empty batch
    fits = _C.paged_decode_workspace_size(100, 16, 8, 16384)
    assert fits <= _C.DECODE_SCRATCH_BYTES < _C.paged_decode_workspace_size(100, 16, 8, 32768)
