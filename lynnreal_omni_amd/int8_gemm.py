"""INT8 x INT8 -> INT32 GEMM with a fused scaled bf16 epilogue, on gfx950 MFMA.

Drop-in for the reference's model/int8_gemm.py: `int8_matmul` keeps its
signature and result (bit-exact bf16, the reference asserts the same equality
against its torch path at script/precompile.py:55-64); `_torch_matmul` is the
reference's torch path (model/int8_gemm.py:84-92).

Differences from the reference, by design:
  * No Triton. The kernel's tile is chosen by shape inside the library;
    `tile=` accepts the reference's tile tuples (BM, BN, BK, warps, stages[,
    group]) and maps (BM, BN) onto the HIP tile of the same shape, or raises
    ValueError. With LYNNREAL_AMD_AUTOTUNE=1 (read at import) the first call of each shape
    times every HIP tile instead and keeps the fastest in memory and in a JSON
    file keyed by library, device and shape (the reference's autotuner and
    tile cache, model/int8_gemm.py:53-81,124-151); every tile computes the
    same bits, so the choice only changes the time.
  * A kernel failure raises instead of silently falling back to torch._int_mm:
    the HIP path is the product, a hidden fallback would mask it.
  * New keyword-only epilogues: activation="gelu_tanh" (GELU-tanh on the bf16
    output) and residual/table/indices/gate_slot (x + gate * y, the reference's
    _gated_residual applied to the GEMM output, model/kernels.py:131-153).
"""
from __future__ import annotations

import functools
import hashlib
import json
import os
import pathlib
import threading

import torch

from . import _lib

_TILES = {
    (256, 256): _lib.TILE_256x256,
    (256, 128): _lib.TILE_256x128,
    (128, 256): _lib.TILE_128x256,
    (128, 128): _lib.TILE_128x128,
    (64, 128): _lib.TILE_64x128,
    (256, 192): _lib.TILE_256x192,
    (256, 80): _lib.TILE_256x80,
    (64, 80): _lib.TILE_64x80,
    (128, 160): _lib.TILE_128x160,
    (192, 256): _lib.TILE_192x256,
}


def _tile_id(tile) -> int:
    if tile is None or tile == "auto":
        return _lib.TILE_AUTO
    if isinstance(tile, str):
        named = {"generic": _lib.TILE_GENERIC, "256x256_w4x2": _lib.TILE_256x256_W4x2,
                 "persistent": _lib.TILE_256x256_PERSISTENT}
        if tile in named:
            return named[tile]
        raise ValueError(f"unknown tile {tile!r}")
    try:
        key = (int(tile[0]), int(tile[1]))
    except (TypeError, ValueError, IndexError):
        raise ValueError(f"tile must be (BM, BN, BK, warps, stages[, group]), got {tile!r}") from None
    if key not in _TILES:
        raise ValueError(f"tile {key} is not one of the HIP tiles {sorted(_TILES)}")
    return _TILES[key]


def _torch_matmul(a, b, row_scale, column_scale, bias):
    """torch._int_mm + fp32 epilogue: the reference's torch path
    (model/int8_gemm.py:84-92) with the same results bit for bit."""
    from .int8 import _int_mm_padded
    out = _int_mm_padded(a, b).float() * row_scale.reshape(-1, 1).float() * column_scale.float()
    if bias is not None:
        out = out + bias.float()
    return out.to(torch.bfloat16)


def _launch(a, b, row_scale, column_scale, bias, out, epilogue, tile, residual=None, table=None,
            indices=None, sequence=0, gate_slot=0, splits=None):
    m, k = a.shape
    n = b.shape[1]
    table_rows = table_width = 0
    if table is not None:
        table_width = table.shape[-1]
        table_rows = table.numel() // table_width
    if tile is None and splits is None and _AUTOTUNE:
        tile = _tuned_tile(a, b, row_scale, column_scale, bias, out, epilogue, residual, table,
                           indices, sequence, gate_slot)
    tile_id = _lib.TILE_AUTO if tile is None else _tile_id(tile)
    splits = 0 if splits is None else int(splits)
    nbytes = _workspace_bytes(m, n, k, splits, tile_id)
    ws, ws_bytes = _lib.workspace(a, nbytes) if nbytes else (None, 0)
    sb0, sb1 = b.stride()
    _lib.call("lr_int8_gemm_ws", a.data_ptr(), b.data_ptr(), sb0, sb1, m, n, k,
              None if row_scale is None else row_scale.data_ptr(),
              None if column_scale is None else column_scale.data_ptr(),
              None if bias is None else bias.data_ptr(), out.data_ptr(), epilogue,
              None if residual is None else residual.data_ptr(),
              None if table is None else table.data_ptr(), table_rows, table_width,
              None if indices is None else indices.data_ptr(), sequence, gate_slot, ws, ws_bytes,
              splits, tile_id, _lib.stream(a))
    return out


# --------------------------------------------------------- autotuning ----
# The candidates: every HIP tile, the library's own choice first, so that a
# tie keeps it.
_CANDIDATES = (None, (256, 256), "persistent", (192, 256), (256, 192), (256, 128), (128, 256),
               (128, 128), (64, 128), (256, 80), (128, 160), (64, 80))
_selected: dict[tuple, object] = {}
_prefixes: dict[int, tuple] = {}


def _autotune_enabled() -> bool:
    """LYNNREAL_AMD_AUTOTUNE as a flag ("", "0" or unset: off)."""
    return os.environ.get("LYNNREAL_AMD_AUTOTUNE", "0") not in ("", "0")


# Read once at import, as the reference reads its LYNNREAL_* switches
# (model/int8_gemm.py:57): an environment lookup costs half a microsecond per call.
_AUTOTUNE = _autotune_enabled()


def _cache_file(key) -> pathlib.Path:
    """The tile cache entry of `key` (model/int8_gemm.py:64-66 keeps its own
    under TRITON_CACHE_DIR; this one lives under LYNNREAL_AMD_CACHE_DIR)."""
    root = pathlib.Path(os.environ.get("LYNNREAL_AMD_CACHE_DIR",
                                       pathlib.Path.home() / ".cache" / "lynnreal_amd"))
    return root / ("int8-" + hashlib.sha256(repr(key).encode()).hexdigest() + ".json")


def _prefix(device: torch.device) -> tuple:
    """What a tuned choice depends on besides the shape: the library's bytes
    and the device (model/int8_gemm.py:107-113 keys on its sources, Triton,
    CUDA and the device's name, capability and SM count)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    prefix = _prefixes.get(index)
    if prefix is None:
        code = hashlib.sha256(_lib.library_path().read_bytes()).hexdigest()
        props = torch.cuda.get_device_properties(index)
        prefix = _prefixes[index] = (code, torch.version.hip, props.name,
                                     getattr(props, "gcnArchName", ""), props.multi_processor_count)
    return prefix


def _encode(tile):
    return list(tile) if isinstance(tile, tuple) else tile


def _decode(saved):
    if isinstance(saved, list):
        saved = tuple(saved)
    return saved if saved in _CANDIDATES else _MISSING


_MISSING = object()


def _tuned_tile(a, b, row_scale, column_scale, bias, out, epilogue, residual, table, indices,
                sequence, gate_slot):
    """The fastest tile for this call's shape, from memory, from the cache
    file, or by timing every candidate once the call has run (graph capture
    takes the library's own choice and records nothing)."""
    m, k = a.shape
    n = b.shape[1]
    key = _prefix(a.device) + (m, n, k, tuple(b.stride()), bias is not None, epilogue)
    tile = _selected.get(key, _MISSING)
    if tile is not _MISSING:
        return tile
    try:
        tile = _decode(json.loads(_cache_file(key).read_text()))
    except (OSError, ValueError, TypeError):
        tile = _MISSING
    if tile is not _MISSING:
        _selected[key] = tile
        return tile
    if torch.cuda.is_current_stream_capturing():
        return None
    args = (a, b, row_scale, column_scale, bias, out, epilogue)
    extra = dict(residual=residual, table=table, indices=indices, sequence=sequence,
                 gate_slot=gate_slot, splits=None)
    best, best_us = None, float("inf")
    for candidate in _CANDIDATES:
        try:
            _launch(*args, candidate if candidate is not None else "auto", **extra)
        except ValueError:
            continue  # a tile this shape does not take
        times = []
        for _ in range(3):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            _launch(*args, candidate if candidate is not None else "auto", **extra)
            end.record()
            end.synchronize()
            times.append(start.elapsed_time(end) * 1e3)
        us = sorted(times)[1]
        if us < best_us:
            best, best_us = candidate, us
    _selected[key] = best
    try:
        path = _cache_file(key)
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_suffix(f".{os.getpid()}.{threading.get_ident()}.tmp")
        tmp.write_text(json.dumps(_encode(best)))
        tmp.replace(path)
    except OSError:
        pass  # a read-only cache directory only loses the record
    return best


@functools.lru_cache(maxsize=4096)
def _workspace_bytes(m, n, k, splits, tile_id) -> int:
    """Workspace bytes of the library's split-K schedule for this shape (0
    when it does not split K), cached per shape."""
    return int(_lib.load().lr_int8_gemm_workspace_size(m, n, k, splits, tile_id))


def _f32_vector(t):
    """t's values as contiguous fp32 in their storage order: t itself when it
    already is (a contiguous [M], [M, 1] or [1, N] fp32 tensor), so that the
    common call converts and copies nothing."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t
    return t.reshape(-1).float().contiguous()


def int8_matmul(a, b, row_scale, column_scale, bias=None, *, tile=None, activation=None,
                residual=None, table=None, indices=None, gate_slot=None, splits=None):
    """bf16(((float)(a @ b) * row_scale) * column_scale + bias) on MFMA.

    a int8 [M, K] contiguous; b int8 [K, N] with any strides (the weight
    layout of Int8Linear, a [K, N] view of [N, K] storage, is the fast path);
    row_scale [M] or [M, 1]; column_scale [N] or [1, N]; bias bf16 [N] or None.
    """
    if a.dtype != torch.int8 or b.dtype != torch.int8 or not a.is_contiguous() or a.shape[1] != b.shape[0]:
        raise ValueError("INT8 GEMM requires contiguous row-major activations and compatible INT8 weights")
    _lib.check_device(a)
    if residual is None:
        _lib.same_device(a, b=b, row_scale=row_scale, column_scale=column_scale, bias=bias)
    else:
        _lib.same_device(a, b=b, row_scale=row_scale, column_scale=column_scale, bias=bias,
                         residual=residual, table=table, indices=indices)
    m, k = a.shape
    n = b.shape[1]
    row_scale = _f32_vector(row_scale)
    column_scale = _f32_vector(column_scale)
    if row_scale.numel() != m or column_scale.numel() != n:
        raise ValueError("row_scale must have M entries and column_scale N entries")
    if bias is not None:
        if bias.dtype != torch.bfloat16:
            raise ValueError("bias must be bfloat16")
        if not bias.is_contiguous():
            bias = bias.contiguous()
        if bias.numel() != n:
            raise ValueError("bias must have N entries")
    output = torch.empty((m, n), device=a.device, dtype=torch.bfloat16)
    if residual is not None:
        if activation is not None:
            raise ValueError("activation and gated residual epilogues are exclusive")
        if table is None or indices is None or gate_slot is None:
            raise ValueError("a gated-residual epilogue needs table, indices and gate_slot")
        if residual.dtype != torch.bfloat16 or table.dtype != torch.bfloat16:
            raise ValueError("residual and table must be bfloat16")
        sequence = residual.shape[-2] if residual.dim() >= 2 else 1
        residual = residual.reshape(m, n).contiguous() if residual.numel() == m * n else None
        if residual is None:
            raise ValueError("residual must have M*N elements")
        table = table.contiguous()
        indices = indices.reshape(-1).contiguous()
        if indices.dtype != torch.int64:
            indices = indices.to(torch.int64)
        if indices.numel() < sequence:
            raise ValueError("indices shorter than the sequence")
        return _launch(a, b, row_scale, column_scale, bias, output, _lib.EPI_GATED_RESIDUAL, tile,
                       residual, table, indices, sequence, int(gate_slot), splits=splits)
    if activation is None:
        epilogue = _lib.EPI_BF16
    elif activation == "gelu_tanh":
        epilogue = _lib.EPI_GELU_TANH
    else:
        raise ValueError(f"unsupported activation {activation!r}")
    return _launch(a, b, row_scale, column_scale, bias, output, epilogue, tile, splits=splits)


def int8_matmul_int32(a, b, *, tile=None, splits=None):
    """Raw int32 accumulators a @ b of the same MFMA kernel (parity/debug)."""
    if a.dtype != torch.int8 or b.dtype != torch.int8 or not a.is_contiguous() or a.shape[1] != b.shape[0]:
        raise ValueError("INT8 GEMM requires contiguous row-major activations and compatible INT8 weights")
    _lib.check_device(a)
    _lib.same_device(a, b=b)
    out = torch.empty((a.shape[0], b.shape[1]), device=a.device, dtype=torch.int32)
    return _launch(a, b, None, None, None, out, _lib.EPI_RAW_INT32, tile, splits=splits)
