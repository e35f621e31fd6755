"""Device-resident handoff plan and K/V row descriptions over the C ABI.

``HandoffPlan`` owns a ``cb_plan``: the job table (target layer, head, kind,
source pairs, window class, RoPE theta sets), the fitted maps pre-packed into
bf16 split terms in MFMA fragment order, and resident RoPE tables. ``Rows``
describes one side of a launch (source page or pool, target pool or output) as
plain device pointers, strides and a token -> row index.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import NamedTuple, Sequence

import numpy as np
import torch

from . import _lib
from .rope import rope_tables

_DTYPES = {torch.bfloat16: _lib.CB_DTYPE_BF16, torch.float16: _lib.CB_DTYPE_F16,
           torch.float32: _lib.CB_DTYPE_F32}


def io_dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"unsupported KV dtype {dtype}; expected bfloat16, float16 or float32") from None


@dataclass
class Rows:
    """One side of a launch: K/V layer buffers, row geometry and token -> row index.

    ``keep`` holds the tensors whose device memory the pointers refer to, so
    they stay alive as long as the description. ``owned`` are the device
    tensors this module allocated for the description (per-layer pointer
    tables): every launch records them on its stream (``hold_for``), so the
    caching allocator does not hand their memory out again while a kernel on
    that stream may still read them, whichever stream allocated them and
    however soon the description is dropped.
    """

    c: _lib.CbRows
    dtype: torch.dtype
    device: torch.device
    keep: list = field(default_factory=list)
    owned: list = field(default_factory=list)

    @property
    def num_layers(self) -> int:
        return self.c.num_layers

    def hold_for(self, stream: torch.cuda.Stream | None) -> None:
        """Keep the owned tables allocated until ``stream``'s queued work is done."""
        if not self.owned:
            return
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        for t in self.owned:
            t.record_stream(s)


def _index_fields(index, block_table, page_size, index_offset, tokens):
    """(kind, pointer, keep) for a token -> row index; validates host-visible sizes."""
    if block_table is not None and index is not None:
        raise ValueError("give either a token index or a block table, not both")
    if block_table is not None:
        if block_table.dtype != torch.int32 or block_table.ndim != 1:
            raise ValueError("block table must be a 1-D int32 tensor")
        if page_size is None or page_size < 1:
            raise ValueError("block table requires page_size >= 1")
        if tokens is not None and (index_offset + tokens + page_size - 1) // page_size > block_table.numel():
            raise ValueError("block table does not cover the block's tokens")
        return _lib.CB_INDEX_BLOCK_TABLE, block_table.data_ptr(), [block_table]
    if index is not None:
        if index.ndim != 1 or index.dtype not in (torch.int32, torch.int64):
            raise ValueError("one-dimensional integer pool indices required")
        if not index.is_contiguous():
            raise ValueError("pool indices must be contiguous")
        if tokens is not None and index_offset + tokens > index.numel():
            raise ValueError("index does not cover the block's tokens")
        kind = _lib.CB_INDEX_I32 if index.dtype == torch.int32 else _lib.CB_INDEX_I64
        return kind, index.data_ptr(), [index]
    return _lib.CB_INDEX_IDENTITY, None, []


def rows_from_page(page: torch.Tensor, *, head_offset: int = 0, tokens=None) -> Rows:
    """Dense ``[2, layers, tokens, heads, head_dim]`` page; row t is token t."""
    if page.ndim != 5 or page.shape[0] != 2:
        raise ValueError("page must be [2,layers,tokens,kv_heads,head_dim]")
    if not page.is_contiguous():
        raise ValueError("page must be contiguous")
    _, layers, n, heads, dim = page.shape
    c = _lib.CbRows()
    c.k_base = page[0].data_ptr()
    c.v_base = page[1].data_ptr()
    c.layer_stride = n * heads * dim
    c.row_stride = heads * dim
    c.rows = n
    c.num_layers = layers
    c.head_offset = head_offset
    c.heads = heads
    c.index_kind = _lib.CB_INDEX_IDENTITY
    return Rows(c, page.dtype, page.device, [page])


def rows_from_layers(k_layers: Sequence[torch.Tensor], v_layers: Sequence[torch.Tensor], *,
                     index=None, block_table=None, page_size=None, index_offset: int = 0,
                     head_offset: int = 0, tokens=None, pointer_cache: dict | None = None) -> Rows:
    """Per-layer ``[rows, heads, head_dim]`` K/V buffers (SGLang pool layout)."""
    if len(k_layers) != len(v_layers) or not k_layers:
        raise ValueError("K and V layer lists must be non-empty and of equal length")
    first = k_layers[0]
    if first.ndim != 3:
        raise ValueError("pool layers must be [rows, kv_heads, head_dim]")
    rows, heads, dim = first.shape
    for t in (*k_layers, *v_layers):
        if t.shape != first.shape or t.dtype != first.dtype or t.device != first.device:
            raise ValueError("pool layers must share shape, dtype and device")
        if not t.is_contiguous():
            raise ValueError("pool layers must be contiguous")
    key = tuple(t.data_ptr() for t in (*k_layers, *v_layers))
    ptrs = pointer_cache.get(key) if pointer_cache is not None else None
    if ptrs is None:
        host = torch.tensor(key, dtype=torch.int64)
        ptrs = host.to(first.device)
        # The table may be read by a kernel on another stream: let the upload
        # land first (once per table when the caller keeps a cache).
        if first.device.type == "cuda":
            torch.cuda.current_stream(first.device).synchronize()
        if pointer_cache is not None:
            pointer_cache.clear()
            pointer_cache[key] = ptrs
    n = len(k_layers)
    kind, idx_ptr, keep = _index_fields(index, block_table, page_size, index_offset, tokens)
    c = _lib.CbRows()
    c.k_layers = ptrs.data_ptr()
    c.v_layers = ptrs.data_ptr() + 8 * n
    c.layer_stride = 0
    c.row_stride = heads * dim
    c.rows = rows
    c.num_layers = n
    c.head_offset = head_offset
    c.heads = heads
    c.index_kind = kind
    c.index = idx_ptr
    c.index_offset = index_offset
    c.page_size = page_size or 0
    return Rows(c, first.dtype, first.device, [ptrs, *keep, *k_layers, *v_layers], owned=[ptrs])


def rows_from_stacked(k: torch.Tensor, v: torch.Tensor, *, index=None, block_table=None,
                      page_size=None, index_offset: int = 0, head_offset: int = 0,
                      tokens=None) -> Rows:
    """Stacked ``[layers, rows, heads, head_dim]`` K and V tensors."""
    if k.ndim != 4 or k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError("stacked K/V must be matching [layers, rows, kv_heads, head_dim]")
    if not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("stacked K/V must be contiguous")
    layers, rows, heads, dim = k.shape
    kind, idx_ptr, keep = _index_fields(index, block_table, page_size, index_offset, tokens)
    c = _lib.CbRows()
    c.k_base = k.data_ptr()
    c.v_base = v.data_ptr()
    c.layer_stride = rows * heads * dim
    c.row_stride = heads * dim
    c.rows = rows
    c.num_layers = layers
    c.head_offset = head_offset
    c.heads = heads
    c.index_kind = kind
    c.index = idx_ptr
    c.index_offset = index_offset
    c.page_size = page_size or 0
    return Rows(c, k.dtype, k.device, [k, v, *keep])


@dataclass(frozen=True)
class ThetaSet:
    """One RoPE configuration: base and optional YaRN scaling dictionary."""

    theta: float
    scaling: dict | None = None

    def key(self):
        return (float(self.theta), tuple(sorted((self.scaling or {}).items())))


def _as_i32(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.int32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


class RequestSpan(NamedTuple):
    """One request of a batched launch (``cb_span``).

    Token ``t`` (``0 <= t < num_tokens``) sits at position
    ``position_start + t``; its source row is the shared source description's
    row of ``u = source_offset + t`` and its target row likewise with
    ``target_offset``. ``prefix_length`` (0: ``position_start + num_tokens``)
    is the whole prefix for sliding-window classes.
    """

    source_offset: int
    target_offset: int
    num_tokens: int
    position_start: int = 0
    prefix_length: int = 0


def _span_array(spans: Sequence[RequestSpan]):
    arr = (_lib.CbSpan * max(1, len(spans)))()
    for i, sp in enumerate(spans):
        sp = RequestSpan(*sp)
        arr[i].source_offset = int(sp.source_offset)
        arr[i].target_offset = int(sp.target_offset)
        arr[i].num_tokens = int(sp.num_tokens)
        arr[i].position_start = int(sp.position_start)
        arr[i].prefix_length = int(sp.prefix_length)
        arr[i].reserved = 0
    return arr


class HandoffPlan:
    """Owner of one device-resident ``cb_plan`` (see ``include/cachebridge_hip.h``).

    Jobs are given per (target layer, target head, kind): ``source_layers`` /
    ``source_heads`` are ``[jobs, s]`` global source indices, ``weights`` is
    ``[jobs, s*D, D]`` fp32 with ``y = x @ W`` and ``biases`` ``[jobs, D]``.
    """

    def __init__(self, *, head_dim: int, dtype: torch.dtype, target_layers: int, target_heads: int,
                 job_target_layer, job_target_head, job_kind, source_layers, source_heads,
                 weights: torch.Tensor, biases: torch.Tensor, thetas: Sequence[ThetaSet],
                 job_source_theta, job_target_theta, job_window=None,
                 window_sizes: Sequence[int] = (0,), max_positions: int = 40960,
                 device: str | torch.device = "cuda"):
        self.lib = _lib.load()
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("the handoff plan lives on a GPU device")
        self.head_dim = int(head_dim)
        self.dtype = dtype
        self.io_code = io_dtype_code(dtype)
        sl = _as_i32(source_layers)
        sh = _as_i32(source_heads)
        if sl.ndim != 2 or sl.shape != sh.shape:
            raise ValueError("source_layers/source_heads must be matching [jobs, support]")
        jobs, support = sl.shape
        self.num_jobs, self.support = jobs, support
        if tuple(weights.shape) != (jobs, support * head_dim, head_dim):
            raise ValueError("weights must be [jobs, support*head_dim, head_dim]")
        if tuple(biases.shape) != (jobs, head_dim):
            raise ValueError("biases must be [jobs, head_dim]")
        if len(window_sizes) < 1 or len(window_sizes) > _lib.CB_MAX_WINDOW_CLASSES:
            raise ValueError("between 1 and 4 window classes are supported")
        self.thetas = list(thetas)
        self.window_sizes = [int(w) for w in window_sizes]
        self.max_positions = int(max_positions)
        arrays = {
            "job_target_layer": _as_i32(job_target_layer),
            "job_target_head": _as_i32(job_target_head),
            "job_kind": _as_i32(job_kind),
            "job_window": _as_i32(job_window if job_window is not None else np.zeros(jobs)),
            "job_source_theta": _as_i32(job_source_theta),
            "job_target_theta": _as_i32(job_target_theta),
            "job_source_layer": sl.reshape(-1).copy(),
            "job_source_head": sh.reshape(-1).copy(),
        }
        for name, arr in arrays.items():
            if name.startswith("job_source_l") or name.startswith("job_source_h"):
                continue
            if arr.shape != (jobs,):
                raise ValueError(f"{name} must have one entry per job")
        w = weights.to(device=self.device, dtype=torch.float32).contiguous()
        b = biases.to(device=self.device, dtype=torch.float32).contiguous()
        cos_all, sin_all = [], []
        for ts in self.thetas:
            c, s = rope_tables(self.head_dim, ts.theta, ts.scaling, self.max_positions)
            cos_all.append(c)
            sin_all.append(s)
        cos_d = torch.stack(cos_all).to(self.device).contiguous()
        sin_d = torch.stack(sin_all).to(self.device).contiguous()
        desc = _lib.CbPlanDesc()
        desc.head_dim = self.head_dim
        desc.support = support
        desc.io_dtype = self.io_code
        desc.num_jobs = jobs
        desc.target_layers = int(target_layers)
        desc.target_heads = int(target_heads)
        for name, arr in arrays.items():
            setattr(desc, name, _ptr(arr))
        desc.d_weight = w.data_ptr()
        desc.d_bias = b.data_ptr()
        desc.num_thetas = len(self.thetas)
        desc.table_positions = self.max_positions
        desc.d_cos = cos_d.data_ptr()
        desc.d_sin = sin_d.data_ptr()
        desc.num_windows = len(self.window_sizes)
        for i, ws in enumerate(self.window_sizes):
            desc.window_size[i] = ws
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            torch.cuda.synchronize(self.device)
            _lib.check(self.lib.cb_plan_create(ctypes.byref(desc), ctypes.byref(handle)))
        self._handle = handle
        self.target_layers = int(target_layers)
        self.target_heads = int(target_heads)
        info = _lib.CbPlanInfo()
        _lib.check(self.lib.cb_plan_get_info(self._handle, ctypes.byref(info)))
        self.info = {name: getattr(info, name) for name, _ in info._fields_}

    def __del__(self):
        handle = getattr(self, "_handle", None)
        if handle is not None and handle.value:
            try:
                self.lib.cb_plan_destroy(handle)
            except Exception:
                pass
            self._handle = None

    def close(self) -> None:
        """Free the plan's device memory (waits for the device first)."""
        if self._handle is not None and self._handle.value:
            torch.cuda.synchronize(self.device)
            self.lib.cb_plan_destroy(self._handle)
        self._handle = None

    def launch(self, source: Rows, target: Rows, *, num_tokens: int, position_start: int,
               prefix_length: int = 0, stream: torch.cuda.Stream | None = None,
               tokens_per_workgroup: int = 0) -> None:
        """Enqueue the fused map + install of one block on ``stream`` (asynchronous)."""
        if self._handle is None:
            raise RuntimeError("plan is closed")
        if source.dtype != self.dtype or target.dtype != self.dtype:
            raise ValueError(f"source/target dtype must be {self.dtype}")
        if source.device != self.device or target.device != self.device:
            raise ValueError("source, target and plan must be on the same device")
        req = _lib.CbRequest()
        req.source = source.c
        req.target = target.c
        req.num_tokens = int(num_tokens)
        req.position_start = int(position_start)
        req.prefix_length = int(prefix_length)
        req.tokens_per_workgroup = int(tokens_per_workgroup)
        _lib.check(self.lib.cb_map_install(self._handle, ctypes.byref(req),
                                           _lib.stream_handle(stream)))
        source.hold_for(stream)
        target.hold_for(stream)

    def workspace_bytes(self, spans: Sequence[RequestSpan]) -> int:
        """Device workspace bytes of a batched launch over ``spans``."""
        if self._handle is None:
            raise RuntimeError("plan is closed")
        total = ctypes.c_int64(0)
        arr = _span_array(spans)
        _lib.check(self.lib.cb_batch_workspace_bytes(self._handle, arr, len(spans), ctypes.byref(total)))
        return int(total.value)

    def launch_batch(self, source: Rows, target: Rows, spans: Sequence[RequestSpan], *,
                     stream: torch.cuda.Stream | None = None) -> None:
        """Enqueue the map + install of every request in ``spans`` as one launch (asynchronous).

        The int32 workspace (source row, target row and position of every kept
        token) comes from torch's caching allocator and is recorded on the
        launch stream, so it is not reused before the launch completes.
        """
        if self._handle is None:
            raise RuntimeError("plan is closed")
        if source.dtype != self.dtype or target.dtype != self.dtype:
            raise ValueError(f"source/target dtype must be {self.dtype}")
        if source.device != self.device or target.device != self.device:
            raise ValueError("source, target and plan must be on the same device")
        arr = _span_array(spans)
        total = ctypes.c_int64(0)
        _lib.check(self.lib.cb_batch_workspace_bytes(self._handle, arr, len(spans), ctypes.byref(total)))
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        workspace = None
        ptr = None
        if total.value > 0:
            with torch.cuda.stream(s):
                workspace = torch.empty(int(total.value), dtype=torch.uint8, device=self.device)
            ptr = workspace.data_ptr()
        _lib.check(self.lib.cb_map_install_batch(self._handle, ctypes.byref(source.c),
                                                 ctypes.byref(target.c), arr, len(spans), ptr,
                                                 int(total.value), _lib.stream_handle(s)))
        source.hold_for(s)
        target.hold_for(s)

    def launch_batch_noalloc(self, source: Rows, target: Rows, spans: Sequence[RequestSpan], *,
                             stream: torch.cuda.Stream | None = None) -> None:
        """``launch_batch`` without allocating: the workspace is the library's fixed per-GPU array.

        Rejects batches beyond ``NOALLOC_MAX_TOKENS`` kept tokens. Calls that
        overlap on one GPU share that array and race; calls on one stream are
        ordered.
        """
        if self._handle is None:
            raise RuntimeError("plan is closed")
        if source.dtype != self.dtype or target.dtype != self.dtype:
            raise ValueError(f"source/target dtype must be {self.dtype}")
        if source.device != self.device or target.device != self.device:
            raise ValueError("source, target and plan must be on the same device")
        arr = _span_array(spans)
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        _lib.check(self.lib.cb_map_install_batch_noalloc(self._handle, ctypes.byref(source.c),
                                                         ctypes.byref(target.c), arr, len(spans),
                                                         _lib.stream_handle(s)))
        source.hold_for(s)
        target.hold_for(s)

    def last_split(self) -> tuple[int, int]:
        """``(pool_chunks, workgroups)`` of this plan's last map launch.

        ``pool_chunks`` is the number of work-pool chunks that launch's
        workgroups claimed dynamically (0: static ranges only).
        """
        chunks, groups = ctypes.c_int32(0), ctypes.c_int32(0)
        _lib.check(self.lib.cb_plan_last_split(self._handle, ctypes.byref(chunks), ctypes.byref(groups)))
        return int(chunks.value), int(groups.value)

    def read_errors(self, stream: torch.cuda.Stream | None = None) -> int:
        """Synchronize ``stream`` and return/clear the device error flags.

        Bit 0: a source row out of range; bit 1: a target row out of range;
        bit 2: a work-pool claim fell past the pool (a host-side
        inconsistency); bit 3: a streaming launch shared its work-pool counter
        pair with another launch in flight (overlapping replays of one graph).
        """
        flags = ctypes.c_int32(0)
        _lib.check(self.lib.cb_plan_read_errors(self._handle, ctypes.byref(flags),
                                                _lib.stream_handle(stream)))
        return int(flags.value)


def copy_rows(src: Rows, dst: Rows, *, num_layers: int, num_tokens: int, row_elements: int,
              error_flag: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None) -> None:
    """Row gather/scatter between two ``Rows`` descriptions (asynchronous)."""
    if src.dtype != dst.dtype:
        raise ValueError("source and destination dtypes differ")
    if src.device != dst.device:
        raise ValueError("source and destination must be on the same device")
    lib = _lib.load()
    flag_ptr = error_flag.data_ptr() if error_flag is not None else None
    _lib.check(lib.cb_copy_rows(ctypes.byref(src.c), ctypes.byref(dst.c), int(num_layers),
                                int(num_tokens), int(row_elements), io_dtype_code(src.dtype),
                                flag_ptr, _lib.stream_handle(stream)))
    src.hold_for(stream)
    dst.hold_for(stream)
