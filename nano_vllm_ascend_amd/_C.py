"""ctypes binding of ``libnvamd.so`` (the C ABI in ``include/nvamd.h``).

The wrappers take torch tensors, check shapes the way the reference's Python
layers do (ValueError on a shape mismatch), pass raw device pointers and the
current HIP stream, and raise if the library reports an error.  There is no
fallback: if the library is missing, every call raises, so a test or bench that
passes has run the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libnvamd.so"

NVAMD_OK = 0
_ERRORS = {-1: "invalid argument", -2: "unsupported configuration", -3: "workspace missing or too small",
           -4: "needs more than the library's static scratch (NVAMD_DECODE_SCRATCH_BYTES)",
           -5: "first use of the static scratch on this device made while the stream is captured; make one "
               "call outside graph capture first"}
DECODE_SCRATCH_BYTES = 64 * 1024 * 1024  # NVAMD_DECODE_SCRATCH_BYTES

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes)
_SIGNATURES = {
    "nvamd_version": (_c_int, []),
    "nvamd_errors_fetch": (_c_int, [_c_ptr, _c_ptr]),
    "nvamd_errors_clear": (_c_int, [_c_ptr]),
    "nvamd_paged_decode_workspace_size": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "nvamd_paged_decode": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_int, _c_ptr,
         _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "nvamd_paged_decode_noalloc": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_int, _c_ptr,
         _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_ptr],
    ),
    "nvamd_paged_decode_fused": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,
         _c_float, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_int, _c_int,
         _c_int, _c_float, _c_int, _c_ptr, _c_size, _c_ptr],
    ),
    "nvamd_kv_cache_write": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_i64, _c_ptr],
    ),
    "nvamd_pack_batch": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_ptr, _c_int, _c_int, _c_ptr,
         _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "nvamd_varlen_prefill": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_float, _c_ptr],
    ),
    "nvamd_paged_prefill": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_int, _c_ptr, _c_ptr,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_ptr],
    ),
    "nvamd_add_rms_norm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_float, _c_ptr]),
    "nvamd_silu_mul": (_c_int, [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_int, _c_int, _c_ptr]),
    "nvamd_argmax_rows": (_c_int, [_c_ptr, _c_i64, _c_int, _c_int, _c_ptr, _c_ptr]),
    "nvamd_skinny_linear_workspace_size": (_c_size, [_c_int, _c_int, _c_int]),
    "nvamd_skinny_linear": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_ptr, _c_float, _c_ptr, _c_ptr, _c_i64, _c_ptr, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_ptr, _c_size, _c_ptr]),
    "nvamd_embed_rows": (
        _c_int, [_c_ptr, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_int, _c_ptr, _c_int, _c_int, _c_ptr]),
    "nvamd_qk_norm_rope": (
        _c_int,
        [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr,
         _c_ptr, _c_ptr, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_float, _c_ptr],
    ),
}

_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    """Names the binding expects the library to export."""
    return sorted(_SIGNATURES)


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m nano_vllm_ascend_amd.build` "
            "(or __graft_entry__.build()); there is no CPU fallback"
        )
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def _check(status: int, name: str) -> None:
    if status == NVAMD_OK:
        return
    if status < 0:
        raise ValueError(f"{name}: {_ERRORS.get(status, 'error')} (status {status})")
    raise RuntimeError(f"{name}: HIP launch failed with hipError_t {status}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream() -> int:
    """hipStream_t of torch's current stream on the current device (the same handle as
    torch.cuda.current_stream().cuda_stream, also under a side stream or graph capture, looked up
    in ~0.3 us instead of ~2.8 us: it is asked for on every eager launch)."""
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require(cond: bool, msg) -> None:
    """Raise ValueError(msg) unless cond; msg may be a callable that builds the message, so a
    passing check formats nothing (these checks run on every eager launch)."""
    if not cond:
        raise ValueError(msg() if callable(msg) else msg)


def _row_stride(t: torch.Tensor) -> int:
    """Element stride between tokens of a [T, heads, D] (or [T, heads*D]) view whose rows are dense."""
    if t.dim() == 3:
        _require(t.stride(2) == 1 and t.stride(1) == t.shape[2], lambda: f"rows of {tuple(t.shape)} are not dense")
    else:
        _require(t.stride(-1) == 1, lambda: f"rows of {tuple(t.shape)} are not dense")
    return t.stride(0)


def _bf16_cuda(name: str, t: torch.Tensor) -> None:
    _require(t.dtype == torch.bfloat16, lambda: f"{name} must be bfloat16, got {t.dtype}")
    _require(t.is_cuda, lambda: f"{name} must be on the GPU")


def version() -> int:
    return int(load().nvamd_version())


# ------------------------------------------------------------------ index errors (device error word)
# Where the reference's indexing raises IndexError (index_copy_ into the KV cache, the RoPE cache
# lookup, the block-table gather), the kernels skip or clamp the access and set a bit in a
# per-device error word.  The runner copies the word to the host with each step's tokens (no extra
# synchronisation) and raises IndexError there.
ERR_SLOT, ERR_POSITION, ERR_CONTEXT, ERR_BLOCK = 1, 2, 4, 8  # NVAMD_ERR_*
_ERR_TEXT = {
    ERR_SLOT: "a slot_mapping entry outside the KV cache (index_copy_, nv/npu/paged_kv_cache.py:68-69)",
    ERR_POSITION: "a position outside the RoPE table (nv/layers/rotary_embedding.py:49-50)",
    ERR_CONTEXT: "a context length its block-table row or the launch's bound cannot hold",
    ERR_BLOCK: "a block-table entry outside the block pool",
}


def describe_index_errors(bits: int) -> str:
    parts = [text for bit, text in _ERR_TEXT.items() if bits & bit]
    unknown = bits & ~sum(_ERR_TEXT)
    if unknown:
        parts.append(f"unknown bits {unknown:#x}")
    return "; ".join(parts)


def clear_index_errors() -> None:
    """Zero the current device's error word (a kernel on the current stream)."""
    _check(load().nvamd_errors_clear(_stream()), "nvamd_errors_clear")


class IndexErrorWord:
    """A host copy of the device's index-error word, fetched on the current stream beside a step's
    other results (pinned memory, so the copy is asynchronous) and checked once they have landed."""

    def __init__(self, host: torch.Tensor | None = None):
        self.host = host if host is not None else torch.zeros(1, dtype=torch.int32, pin_memory=True)

    def fetch(self) -> None:
        _check(load().nvamd_errors_fetch(self.host.data_ptr(), _stream()), "nvamd_errors_fetch")

    def raise_if_set(self) -> None:
        """Call after the copy has landed (the step's tokens were read)."""
        bits = int(self.host[0])
        if bits:
            self.host.zero_()
            clear_index_errors()
            raise IndexError(f"index out of range in the step's kernels: {describe_index_errors(bits)} "
                             f"(error word {bits:#x})")


def index_errors() -> int:
    """The current device's error word, read synchronously (tests and debugging)."""
    word = IndexErrorWord()
    word.fetch()
    torch.cuda.current_stream().synchronize()
    return int(word.host[0])


# ------------------------------------------------------------------ optional host-side range checks
# The kernels never read or write outside their buffers, but where the reference's torch indexing
# (index_select of the RoPE cache, index_copy_ into the KV cache, the block-table gather) would
# raise on an index out of range they clamp, skip or truncate instead.  With range checks on
# (set_range_checks(True), or NVAMD_CHECK_RANGES=1 in the environment) the eager wrappers read the
# indices back to the host and raise IndexError first.  That costs a device-to-host copy per call,
# so it is a debugging aid, off by default; calls made while a graph is being captured are not
# checked (a capture cannot synchronise).
_range_checks = os.environ.get("NVAMD_CHECK_RANGES", "") not in ("", "0")


def set_range_checks(enabled: bool) -> bool:
    """Turn the host-side range checks on or off; returns the previous setting."""
    global _range_checks
    prev, _range_checks = _range_checks, bool(enabled)
    return prev


def _checking() -> bool:
    return _range_checks and not (torch.cuda.is_available() and torch.cuda.is_current_stream_capturing())


def check_positions(positions: torch.Tensor, max_positions: int) -> None:
    """RoPE rows are index_select-ed by position (nv/layers/rotary_embedding.py:44-55)."""
    pos = positions.detach().reshape(-1).cpu()
    if pos.numel() and (int(pos.min()) < 0 or int(pos.max()) >= max_positions):
        raise IndexError(f"position out of range [0, {max_positions}) of the RoPE table: "
                         f"min {int(pos.min())}, max {int(pos.max())}")


def check_slots(slot_mapping: torch.Tensor, num_slots: int) -> None:
    """K/V rows are index_copy_-ed at their slots (nv/npu/paged_kv_cache.py:68-69); -1 marks a padding
    row that is not stored (an extension the reference never emits)."""
    sl = slot_mapping.detach().reshape(-1).cpu()
    if sl.numel() and (int(sl.min()) < -1 or int(sl.max()) >= num_slots):
        raise IndexError(f"slot out of range [0, {num_slots}) (or -1 for padding): "
                         f"min {int(sl.min())}, max {int(sl.max())}")


def check_paged_context(block_tables: torch.Tensor, context_lens: torch.Tensor, num_blocks: int, block_size: int,
                        max_context_len: int | None = None) -> None:
    """Every context fits its bound and its block-table row, and the entries it reads name pool blocks
    (the reference gathers K/V through the table, nv/layers/npu_paged_attention.py:89-99)."""
    ctx = context_lens.detach().reshape(-1).cpu().long()
    bt = block_tables.detach().cpu().long()
    width = bt.shape[1] * block_size
    for i, c in enumerate(ctx.tolist()):
        if c < 0 or c > width or (max_context_len is not None and c > max_context_len):
            raise IndexError(f"context length {c} of row {i} is outside [0, min({width}, "
                             f"{max_context_len if max_context_len is not None else width})]")
        used = bt[i, : -(-c // block_size)]
        if used.numel() and (int(used.min()) < 0 or int(used.max()) >= num_blocks):
            raise IndexError(f"block-table row {i} names a block outside [0, {num_blocks}): {used.tolist()}")


def paged_decode_workspace_size(max_batch: int, num_heads: int, num_kv_heads: int, max_context_len: int) -> int:
    return int(load().nvamd_paged_decode_workspace_size(max_batch, num_heads, num_kv_heads, max_context_len))


def alloc_paged_decode_workspace(max_batch: int, num_heads: int, num_kv_heads: int, max_context_len: int,
                                 device) -> torch.Tensor:
    """Zero-filled workspace (the kernel keeps its counters at zero between calls)."""
    nbytes = paged_decode_workspace_size(max_batch, num_heads, num_kv_heads, max_context_len)
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def paged_decode(out: torch.Tensor, q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float, max_context_len: int,
                 workspace: torch.Tensor) -> torch.Tensor:
    """out[i,h] = softmax(q[i,h] K^T * scale) V over the paged context of sequence i.

    q/out: [B, Hq, 128] bf16 (dense rows, any token stride); caches
    [NB, block_size, Hkv, 128] bf16; block_tables int32 [B, W]; context_lens
    int32 [B] on the device; max_context_len bounds every context_lens entry.
    """
    lib = load()
    args = _decode_args(out, q, key_cache, value_cache, block_tables, context_lens, scale, max_context_len)
    status = lib.nvamd_paged_decode(*args, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                                    _stream())
    _check(status, "nvamd_paged_decode")
    return out


def paged_decode_noalloc(out: torch.Tensor, q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                         block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                         max_context_len: int) -> torch.Tensor:
    """``paged_decode`` without a workspace: the library's static per-GPU scratch serves as one.

    Raises ValueError when the call needs more than DECODE_SCRATCH_BYTES
    (paged_decode_workspace_size of its sizes), or when the first call on a device is made under
    graph capture (the first call clears the scratch's counters, which capture would only record).
    Calls that overlap on one GPU share the scratch and race.
    """
    lib = load()
    args = _decode_args(out, q, key_cache, value_cache, block_tables, context_lens, scale, max_context_len)
    _check(lib.nvamd_paged_decode_noalloc(*args, _stream()), "nvamd_paged_decode_noalloc")
    return out


def _decode_args(out, q, key_cache, value_cache, block_tables, context_lens, scale, max_context_len) -> tuple:
    """Checked arguments of the decode entry points, up to the workspace."""
    _bf16_cuda("q", q)
    _bf16_cuda("out", out)
    _bf16_cuda("key_cache", key_cache)
    _bf16_cuda("value_cache", value_cache)
    _require(q.dim() == 3 and out.shape == q.shape,
             lambda: f"q/out shape mismatch: {tuple(q.shape)} vs {tuple(out.shape)}")
    _require(key_cache.dim() == 4 and key_cache.shape == value_cache.shape, "key/value cache shape mismatch")
    _require(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    nb, bs, hkv, d = key_cache.shape
    b, hq, dq = q.shape
    _require(dq == d, lambda: f"head_dim mismatch {dq} vs {d}")
    _require(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and block_tables.shape[0] == b,
             "block_tables must be int32 [B, W]")
    _require(block_tables.stride(1) == 1, "block_tables rows must be dense")
    _require(context_lens.dtype == torch.int32 and context_lens.numel() == b and context_lens.is_cuda,
             "context_lens must be int32 [B] on the device")
    _require(context_lens.is_contiguous(), "context_lens must be contiguous")
    if _checking():
        check_paged_context(block_tables, context_lens, nb, bs, int(max_context_len))
    return (out.data_ptr(), _row_stride(out), q.data_ptr(), _row_stride(q), key_cache.data_ptr(),
            value_cache.data_ptr(), nb, bs, block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
            context_lens.data_ptr(), b, hq, hkv, d, float(scale), int(max_context_len))


def paged_decode_fused(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       q_weight: torch.Tensor, k_weight: torch.Tensor, positions: torch.Tensor,
                       cos_sin: torch.Tensor, eps: float, key_cache: torch.Tensor, value_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, block_tables: torch.Tensor, context_lens: torch.Tensor,
                       scale: float, max_context_len: int, workspace: torch.Tensor) -> torch.Tensor:
    """One decode step of attention: qk_norm_rope (with the KV store) then paged_decode, in one launch.

    q: raw [B, Hq, 128] and k, v: raw [B, Hkv, 128] rows of the new tokens (views into the
    projection output are fine; they are not modified).  Writes out and the caches only.
    slot_mapping[i] must be the cache slot of row positions[i] of sequence i (decode metadata).
    """
    lib = load()
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        _bf16_cuda(name, t)
    _require(q.dim() == 3 and out.shape == q.shape,
             lambda: f"q/out shape mismatch: {tuple(q.shape)} vs {tuple(out.shape)}")
    _require(k.dim() == 3 and k.shape == v.shape and k.shape[0] == q.shape[0], "k/v must be [B, Hkv, D]")
    _require(key_cache.dim() == 4 and key_cache.shape == value_cache.shape, "key/value cache shape mismatch")
    _require(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    nb, bs, hkv, d = key_cache.shape
    b, hq, dq = q.shape
    _require(dq == d and k.shape[1:] == (hkv, d),
             lambda: f"head shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}")
    _require(q_weight.dtype == torch.bfloat16 and k_weight.dtype == torch.bfloat16, "norm weights must be bf16")
    _require(q_weight.numel() == d and k_weight.numel() == d, "norm weights must have head_dim elements")
    _require(q_weight.is_contiguous() and k_weight.is_contiguous(), "norm weights must be contiguous")
    _require(positions.dtype == torch.int64 and positions.numel() == b and positions.is_cuda,
             "positions must be int64 [B] on the device")
    _require(cos_sin.dtype == torch.float32 and cos_sin.dim() == 2 and cos_sin.shape[1] == d and cos_sin.is_cuda
             and cos_sin.is_contiguous(), "cos_sin must be contiguous fp32 [max_positions, head_dim]")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.numel() == b and slot_mapping.is_cuda,
             "slot_mapping must be int64 [B] on the device")
    _require(block_tables.dtype == torch.int32 and block_tables.dim() == 2 and block_tables.shape[0] == b,
             "block_tables must be int32 [B, W]")
    _require(block_tables.stride(1) == 1, "block_tables rows must be dense")
    _require(context_lens.dtype == torch.int32 and context_lens.numel() == b and context_lens.is_cuda
             and context_lens.is_contiguous(), "context_lens must be int32 [B] on the device")
    if _checking():
        check_paged_context(block_tables, context_lens, nb, bs, int(max_context_len))
        check_positions(positions, cos_sin.shape[0])
        check_slots(slot_mapping, nb * bs)
    status = lib.nvamd_paged_decode_fused(
        out.data_ptr(), _row_stride(out), q.data_ptr(), _row_stride(q), k.data_ptr(), _row_stride(k),
        v.data_ptr(), _row_stride(v), q_weight.data_ptr(), k_weight.data_ptr(), positions.contiguous().data_ptr(),
        cos_sin.data_ptr(), cos_sin.shape[0], float(eps), key_cache.data_ptr(), value_cache.data_ptr(), nb, bs,
        slot_mapping.contiguous().data_ptr(), block_tables.data_ptr(), block_tables.stride(0),
        block_tables.shape[1], context_lens.data_ptr(), b, hq, hkv, d, float(scale), int(max_context_len),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream(),
    )
    _check(status, "nvamd_paged_decode_fused")
    return out


def kv_cache_write(key_states: torch.Tensor, value_states: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """cache_flat[slot_mapping[t]] = kv[t] for the K and the V cache of one layer."""
    lib = load()
    _bf16_cuda("key_states", key_states)
    _bf16_cuda("value_states", value_states)
    _require(key_states.shape == value_states.shape and key_states.dim() == 3, "k/v shape mismatch")
    t, hkv, d = key_states.shape
    _require(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    _require(key_cache.shape[-2:] == (hkv, d), lambda: f"kv shape mismatch: got {tuple(key_states.shape)}")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.numel() == t and slot_mapping.is_cuda,
             f"slot_mapping numel {slot_mapping.numel()} != total_tokens {t}")
    num_slots = key_cache.numel() // (hkv * d)
    if _checking():
        check_slots(slot_mapping, num_slots)
    status = lib.nvamd_kv_cache_write(
        key_states.data_ptr(), _row_stride(key_states), value_states.data_ptr(), _row_stride(value_states),
        key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.contiguous().data_ptr(), t, hkv, d, num_slots,
        _stream(),
    )
    _check(status, "nvamd_kv_cache_write")


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                 positions: torch.Tensor, cos_sin: torch.Tensor, eps: float,
                 v: torch.Tensor | None = None, key_cache: torch.Tensor | None = None,
                 value_cache: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None) -> None:
    """In place: q, k <- RoPE(RMSNorm_head(x) * w); optionally store post-RoPE k and v in the caches."""
    lib = load()
    _bf16_cuda("q", q)
    _bf16_cuda("k", k)
    _require(q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0], "q/k must be [T, heads, D]")
    t, hq, d = q.shape
    hkv = k.shape[1]
    _require(k.shape[2] == d, "q/k head_dim mismatch")
    _require(q_weight.dtype == torch.bfloat16 and k_weight.dtype == torch.bfloat16, "norm weights must be bf16")
    _require(q_weight.numel() == d and k_weight.numel() == d, "norm weights must have head_dim elements")
    _require(positions.dtype == torch.int64 and positions.numel() == t and positions.is_cuda,
             "positions must be int64 [T] on the device")
    _require(cos_sin.dtype == torch.float32 and cos_sin.dim() == 2 and cos_sin.shape[1] == d and cos_sin.is_cuda,
             "cos_sin must be fp32 [max_positions, head_dim]")
    store = key_cache is not None
    num_slots = 0
    if store:
        _require(v is not None and value_cache is not None and slot_mapping is not None, "store needs v, caches, slots")
        _bf16_cuda("v", v)
        _require(v.shape == k.shape, "k/v shape mismatch")
        _require(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
        _require(slot_mapping.dtype == torch.int64 and slot_mapping.numel() == t, "slot_mapping must be int64 [T]")
        num_slots = key_cache.numel() // (hkv * d)
    if _checking():
        check_positions(positions, cos_sin.shape[0])
        if store:
            check_slots(slot_mapping, num_slots)
    status = lib.nvamd_qk_norm_rope(
        q.data_ptr(), _row_stride(q), k.data_ptr(), _row_stride(k), _ptr(v), _row_stride(v) if store else 0,
        q_weight.data_ptr(), k_weight.data_ptr(), positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping.contiguous()) if store else None, num_slots,
        t, hq, hkv, d, float(eps), _stream(),
    )
    _check(status, "nvamd_qk_norm_rope")


def pack_batch(desc: torch.Tensor, batch: int, updates: torch.Tensor | None, num_updates: int,
               token_ids: torch.Tensor | None, mirror: torch.Tensor, block_size: int,
               block_tables: torch.Tensor | None = None, context_lens: torch.Tensor | None = None,
               slot_mapping: torch.Tensor | None = None, positions: torch.Tensor | None = None,
               cu_seqlens: torch.Tensor | None = None, last_token_indices: torch.Tensor | None = None,
               input_ids: torch.Tensor | None = None) -> None:
    """Expand per-sequence descriptors into the packed-batch metadata on the GPU (see nvamd.h)."""
    lib = load()
    _require(desc.dtype == torch.int32 and desc.is_cuda and desc.numel() >= 5 * batch, "desc must be int32 [5, B]")
    _require(mirror.dtype == torch.int32 and mirror.dim() == 2 and mirror.is_contiguous(), "mirror must be int32 2-D")
    if block_tables is not None:
        _require(block_tables.dtype == torch.int32 and block_tables.stride(1) == 1 and block_tables.shape[0] >= batch,
                 "block_tables must be int32 [B, W] with dense rows")
    for name, t, dt in (("context_lens", context_lens, torch.int32), ("slot_mapping", slot_mapping, torch.int64),
                        ("positions", positions, torch.int64), ("cu_seqlens", cu_seqlens, torch.int32),
                        ("last_token_indices", last_token_indices, torch.int64),
                        ("input_ids", input_ids, torch.int64)):
        if t is not None:
            _require(t.dtype == dt and t.is_cuda and t.is_contiguous(),
                     lambda: f"{name} must be a contiguous {dt} GPU tensor")
    status = lib.nvamd_pack_batch(
        desc.data_ptr(), batch, _ptr(updates), num_updates, _ptr(token_ids), mirror.data_ptr(), mirror.shape[1],
        mirror.shape[0], block_size, _ptr(block_tables), block_tables.stride(0) if block_tables is not None else 0,
        block_tables.shape[1] if block_tables is not None else 0, _ptr(context_lens), _ptr(slot_mapping),
        _ptr(positions), _ptr(cu_seqlens), _ptr(last_token_indices), _ptr(input_ids), _stream(),
    )
    _check(status, "nvamd_pack_batch")


def varlen_prefill(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                   max_q_len: int, scale: float) -> torch.Tensor:
    """Dense causal varlen attention: q/out [T, Hq, 128], k/v [T, Hkv, 128], cu_seqlens_q int32 [B+1] (device)."""
    lib = load()
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        _bf16_cuda(name, t)
        _require(t.dim() == 3, lambda: f"{name} must be [T, heads, D]")
    _require(out.shape == q.shape, "q/out shape mismatch")
    _require(k.shape == v.shape and k.shape[0] == q.shape[0], lambda: f"k/v token mismatch: q={tuple(q.shape)} "
             f"k={tuple(k.shape)} v={tuple(v.shape)}")
    _require(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.is_cuda and cu_seqlens_q.is_contiguous(),
             "cu_seqlens_q must be int32 on the device")
    n_seqs = cu_seqlens_q.numel() - 1
    status = lib.nvamd_varlen_prefill(
        out.data_ptr(), _row_stride(out), q.data_ptr(), _row_stride(q), k.data_ptr(), _row_stride(k),
        v.data_ptr(), _row_stride(v), cu_seqlens_q.data_ptr(), n_seqs, int(max_q_len), q.shape[1], k.shape[1],
        q.shape[2], float(scale), _stream(),
    )
    _check(status, "nvamd_varlen_prefill")
    return out


def paged_prefill(out: torch.Tensor, q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                  block_tables: torch.Tensor, cu_seqlens_q: torch.Tensor, kv_lens: torch.Tensor, max_q_len: int,
                  scale: float) -> torch.Tensor:
    """Prefix-hit prefill: queries are the last q_len of kv_len positions, keys read through the cache pages."""
    lib = load()
    for name, t in (("q", q), ("out", out), ("key_cache", key_cache), ("value_cache", value_cache)):
        _bf16_cuda(name, t)
    _require(out.shape == q.shape and q.dim() == 3, "q/out shape mismatch")
    _require(key_cache.dim() == 4 and key_cache.shape == value_cache.shape, "key/value cache shape mismatch")
    _require(key_cache.is_contiguous() and value_cache.is_contiguous(), "caches must be contiguous")
    _require(block_tables.dtype == torch.int32 and block_tables.stride(1) == 1, "block_tables must be int32 [B, W]")
    _require(cu_seqlens_q.dtype == torch.int32 and kv_lens.dtype == torch.int32 and kv_lens.is_cuda,
             "cu_seqlens_q / kv_lens must be int32 on the device")
    nb, bs, hkv, d = key_cache.shape
    n_seqs = cu_seqlens_q.numel() - 1
    _require(kv_lens.numel() >= n_seqs and block_tables.shape[0] >= n_seqs, "per-sequence metadata too short")
    if _checking():
        check_paged_context(block_tables[:n_seqs], kv_lens[:n_seqs], nb, bs)
    status = lib.nvamd_paged_prefill(
        out.data_ptr(), _row_stride(out), q.data_ptr(), _row_stride(q), key_cache.data_ptr(), value_cache.data_ptr(),
        nb, bs, block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1], cu_seqlens_q.data_ptr(),
        kv_lens.data_ptr(), n_seqs, int(max_q_len), q.shape[1], hkv, d, float(scale), _stream(),
    )
    _check(status, "nvamd_paged_prefill")
    return out


def add_rms_norm(delta: torch.Tensor | None, residual: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
                 eps: float) -> torch.Tensor:
    """residual += delta (if given); out = RMSNorm(residual) * weight.  Rows of any multiple of 8 bf16
    elements."""
    lib = load()
    _bf16_cuda("residual", residual)
    _bf16_cuda("out", out)
    _require(residual.is_contiguous() and out.is_contiguous() and out.shape == residual.shape, "rows must be dense")
    _require(weight.dtype == torch.bfloat16 and weight.numel() == residual.shape[-1], "weight must be bf16 [hidden]")
    if delta is not None:
        _require(delta.shape == residual.shape and delta.is_contiguous() and delta.dtype == torch.bfloat16,
                 "delta must match residual")
    hidden = residual.shape[-1]
    status = lib.nvamd_add_rms_norm(_ptr(delta), residual.data_ptr(), weight.data_ptr(), out.data_ptr(),
                                    residual.numel() // hidden, hidden, float(eps), _stream())
    _check(status, "nvamd_add_rms_norm")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate_up[:, :I]) * gate_up[:, I:] for a [T, 2I] bf16 projection output."""
    lib = load()
    _bf16_cuda("gate_up", gate_up)
    t, two_i = gate_up.shape
    inter = two_i // 2
    out = torch.empty((t, inter), dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    status = lib.nvamd_silu_mul(gate_up.data_ptr(), _row_stride(gate_up), out.data_ptr(), _row_stride(out), t, inter,
                                _stream())
    _check(status, "nvamd_silu_mul")
    return out


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """First index of each row's maximum (int64 [rows]) of a bf16 [rows, vocab] tensor."""
    lib = load()
    _bf16_cuda("logits", logits)
    rows, vocab = logits.shape
    out = torch.empty(rows, dtype=torch.int64, device=logits.device) if out is None else out
    _require(out.dtype == torch.int64 and out.numel() >= rows, "out must be int64 [rows]")
    status = lib.nvamd_argmax_rows(logits.data_ptr(), _row_stride(logits), rows, vocab, out.data_ptr(), _stream())
    _check(status, "nvamd_argmax_rows")
    return out


SKINNY_MAX_ROWS = 128  # rows the skinny projection kernels take (decode batches)
EPI_STORE, EPI_SILU, EPI_RESID = 0, 1, 2


def skinny_linear_workspace_size(n: int, k: int, epilogue: int = EPI_STORE) -> int:
    """Bytes of zero-filled workspace a skinny projection of this shape needs (0: none)."""
    return int(load().nvamd_skinny_linear_workspace_size(n, k, epilogue))


GEMM_X_TILED = 1
GEMM_Y_TILED = 2


def is_tiled(t: torch.Tensor) -> bool:
    """A tiled matrix is a contiguous [rows/16, cols/32, 512] tensor (the skinny GEMM's operand order)."""
    return t.dim() == 3 and t.shape[2] == 512


def tile(a: torch.Tensor) -> torch.Tensor:
    """Row-major [R, C] (C % 32 == 0) -> tiled [ceil(R/16), C/32, 512]: 16 x 32 tiles, row-tile major,
    element (r, c) of a tile at 128 * (c // 8) + 8 * r + c % 8.  Padding rows are zero."""
    _require(a.dim() == 2 and a.shape[1] % 32 == 0, "tile() takes [R, C] with C % 32 == 0")
    r, c = a.shape
    rp = -(-r // 16) * 16
    if rp != r:
        a = torch.cat([a, a.new_zeros(rp - r, c)])
    return a.reshape(rp // 16, 16, c // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(rp // 16, c // 32, 512).contiguous()


def untile(t: torch.Tensor, rows: int | None = None) -> torch.Tensor:
    """Tiled [R/16, C/32, 512] -> row-major [rows, C] (a copy; rows defaults to R)."""
    _require(is_tiled(t), "untile() takes a tiled [R/16, C/32, 512] tensor")
    rt, ct, _ = t.shape
    a = t.reshape(rt, ct, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(rt * 16, ct * 32)
    return (a if rows is None else a[:rows]).contiguous()


def tiled_empty(rows: int, cols: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """Uninitialised tiled storage for a [rows, cols] matrix (rows padded to a multiple of 16)."""
    return torch.empty((-(-rows // 16), cols // 32, 512), dtype=dtype, device=device)


def skinny_linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None, *, epilogue: int = EPI_STORE,
                  x_ssq: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                  y_ssq: torch.Tensor | None = None, workspace: torch.Tensor | None = None, m: int | None = None,
                  y_tiled: bool = False) -> torch.Tensor:
    """Decode-batch projection x[M, K] @ W^T (M <= 128) with an optional RMSNorm prologue and a store,
    SiLU*mul or residual-add epilogue (one HIP launch).  Returns the output (the residual for EPI_RESID).

    w is the weight tiled (``tile(W)``; SILU: the fused [2I, K] gate/up weight).  x is row-major
    [M, K] or tiled (then ``m`` gives the valid rows); with ``y_tiled`` the output (the residual
    for EPI_RESID) is tiled with 16 * ceil(M/16) rows."""
    lib = load()
    _bf16_cuda("x", x)
    _bf16_cuda("w", w)
    _require(is_tiled(w), "w must be tiled: tile(W)")
    x_tiled = is_tiled(x)
    if x_tiled:
        _require(m is not None and 0 <= m <= 16 * x.shape[0], "a tiled x needs m <= its padded rows")
        _require(m <= 16 or x.shape[0] >= 2, "a tiled x of more than 16 rows holds 32")
        k = 32 * x.shape[1]
    else:
        m, k = x.shape
    _require(32 * w.shape[1] == k, "w must be tiled [N/16, K/32, 512]")
    n = 8 * w.shape[0] if epilogue == EPI_SILU else 16 * w.shape[0]
    if epilogue == EPI_RESID:
        _require(out is not None, "the residual epilogue updates `out` in place")
        _require(y_ssq is not None and y_ssq.dtype == torch.float32 and y_ssq.is_contiguous()
                 and y_ssq.numel() >= m * (n // 32), "y_ssq must be fp32 [M, N/32]")
    if y_tiled:
        out = tiled_empty(max(m, 1), n, x.device) if out is None else out
        _require(is_tiled(out) and out.dtype == torch.bfloat16 and out.shape[1] * 32 == n
                 and 16 * out.shape[0] >= m and (m <= 16 or out.shape[0] >= 2), "out must be tiled bf16 [M, N]")
    else:
        out = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out
        _require(out.shape == (m, n) and out.dtype == torch.bfloat16 and out.stride(1) == 1,
                 "out must be bf16 [M, N]")
    if x_ssq is not None:
        _require(norm_weight is not None and norm_weight.dtype == torch.bfloat16 and norm_weight.numel() == k,
                 "norm_weight must be bf16 [K]")
        _require(x_ssq.dtype == torch.float32 and x_ssq.is_contiguous() and x_ssq.numel() >= m * (k // 32),
                 "x_ssq must be fp32 [M, K/32]")
    need = skinny_linear_workspace_size(n, k, epilogue) if n % 32 == 0 and k % 256 == 0 else 0
    if need and workspace is None:
        workspace = torch.zeros(need, dtype=torch.uint8, device=x.device)
    flags = (GEMM_X_TILED if x_tiled else 0) | (GEMM_Y_TILED if y_tiled else 0)
    status = lib.nvamd_skinny_linear(
        x.data_ptr(), 0 if x_tiled else _row_stride(x), _ptr(x_ssq), _ptr(norm_weight), float(eps), w.data_ptr(),
        out.data_ptr(), 0 if y_tiled else out.stride(0), _ptr(y_ssq), int(epilogue), flags, m, n, k,
        _ptr(workspace), workspace.numel() if workspace is not None else 0, _stream())
    _check(status, "nvamd_skinny_linear")
    return out


def linear(x: torch.Tensor, w_tiled: torch.Tensor, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None) -> torch.Tensor:
    """x[M, K] @ W[N, K]^T in bf16 for M <= 128 (HIP skinny GEMM; w_tiled = tile(W))."""
    return skinny_linear(x, w_tiled, out, workspace=workspace)


def linear_silu_mul(x: torch.Tensor, w_gate_up_tiled: torch.Tensor, out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """silu(x @ W[:I]^T) * (x @ W[I:]^T) in bf16 for M <= 128 (one HIP launch; W the [2I, K] gate/up
    weight, passed as tile(W))."""
    _require(w_gate_up_tiled.shape[0] % 2 == 0, "the gate/up weight must be [2I, K]")
    return skinny_linear(x, w_gate_up_tiled, out, epilogue=EPI_SILU, workspace=workspace)


def embed_rows(ids: torch.Tensor, table: torch.Tensor, out: torch.Tensor | None = None,
               ssq: torch.Tensor | None = None, out_tiled: bool = False) -> torch.Tensor:
    """table[ids] (zero rows for ids outside the vocab) and, if given, per-32-column sums of squares.
    With ``out_tiled`` the rows are written tiled (16 * ceil(rows/16) padded rows, padding untouched)."""
    lib = load()
    _bf16_cuda("table", table)
    _require(ids.dtype == torch.int64 and ids.is_cuda and ids.is_contiguous(), "ids must be int64 on the GPU")
    rows = ids.numel()
    vocab, hidden = table.shape
    if out_tiled:
        out = tiled_empty(max(rows, 1), hidden, table.device) if out is None else out
        _require(is_tiled(out) and out.dtype == torch.bfloat16 and out.shape[1] * 32 == hidden
                 and 16 * out.shape[0] >= rows, "out must be tiled bf16 [rows, hidden]")
    else:
        out = torch.empty((rows, hidden), dtype=table.dtype, device=table.device) if out is None else out
        _require(out.shape == (rows, hidden) and out.dtype == torch.bfloat16, "out must be bf16 [rows, hidden]")
    if ssq is not None:
        _require(ssq.dtype == torch.float32 and ssq.is_contiguous() and ssq.numel() >= rows * (hidden // 32),
                 "ssq must be fp32 [rows, hidden/32]")
    status = lib.nvamd_embed_rows(ids.data_ptr(), table.data_ptr(), _row_stride(table), vocab, out.data_ptr(),
                                  0 if out_tiled else _row_stride(out), int(out_tiled), _ptr(ssq), rows, hidden,
                                  _stream())
    _check(status, "nvamd_embed_rows")
    return out
