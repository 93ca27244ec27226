"""Tensor-level entry points of the paged KV-cache kernels.

Each function validates shapes on the host, then passes raw device pointers, element
strides and the current HIP stream through the C ABI (``include/mipaged.h``). Nothing
here computes on the CPU: tensors that are not on a ROCm device raise.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _native

_DTYPE_CODES = {torch.float32: _native.MIP_F32, torch.float16: _native.MIP_F16, torch.bfloat16: _native.MIP_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported KV dtype {dtype}; expected float32, float16 or bfloat16") from None


def _require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "the paged KV-cache kernels run only on a ROCm GPU device (got a tensor on "
                f"{t.device}); there is no CPU path"
            )


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    """Handle of the current stream on ``device`` (``torch.cuda.current_stream(device).cuda_stream``)."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


class PreparedCall:
    """One validated C-ABI call with its argument tuple fixed (pointers, strides, stream).

    Calling it re-launches the kernel on the same buffers with no Python-side checks, for
    loops over static buffers (timing, serving loops). The stream is the one current when
    the call was prepared: a call meant for a graph must be prepared inside the capture.
    The tensors passed to the ``prepare_*`` function must stay alive and in place while it
    is used.
    """

    __slots__ = ("_fn", "_args", "_what", "keep")

    def __init__(self, fn, args: tuple, what: str, keep: tuple = ()) -> None:
        self._fn, self._args, self._what, self.keep = fn, args, what, keep

    def __call__(self) -> None:
        st = self._fn(*self._args)
        if st:
            _native.check(st, self._what)


def _noop() -> None:
    return None


def prepare_kv_append(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      slot_mapping: torch.Tensor):
    """Validate a :func:`kv_append` call once; returns a :class:`PreparedCall` (or a no-op for N = 0)."""
    _require_device(k_cache, v_cache, k, v, slot_mapping)
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous [num_blocks, Hkv, block_size, D] tensors of one shape")
    nb, hkv, bs, d = k_cache.shape
    if k.dim() != 3 or k.shape != v.shape or k.shape[1:] != (hkv, d):
        raise ValueError(f"k/v must be [N, {hkv}, {d}], got {tuple(k.shape)} and {tuple(v.shape)}")
    if k.dtype != k_cache.dtype or v.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError("k, v and the cache must share one dtype")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("the last (head_dim) dimension of k/v must be contiguous")
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.shape[0] != k.shape[0]:
        raise ValueError("slot_mapping must be int64 [N]")
    if not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous")
    n = k.shape[0]
    if n == 0:
        return _noop
    lib = _native.load()
    args = (k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), nb, slot_mapping.data_ptr(), n, hkv, d, bs,
            dtype_code(k_cache.dtype), _stream_ptr(k_cache.device))
    return PreparedCall(lib.mip_kv_append, args, "mip_kv_append", (k_cache, v_cache, k, v, slot_mapping))


def kv_append(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Write token i's K/V rows (``k[i, h, :]``) to pool slot ``slot_mapping[i]``.

    ``k_cache``/``v_cache``: one layer of the pool, ``[num_blocks + 1, Hkv, block_size, D]``
    contiguous. ``k``/``v``: ``[N, Hkv, D]`` with any token/head strides and a contiguous
    last dimension. ``slot_mapping``: int64 ``[N]``, ``block * block_size + offset``.
    Follows engine/kv_cache.py:613-614 and :286-289 (bit-exact data movement).
    """
    prepare_kv_append(k_cache, v_cache, k, v, slot_mapping)()


def prepare_rope_kv_append(q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                           sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           slot_mapping: torch.Tensor):
    """Validate a :func:`rope_kv_append` call once; returns a :class:`PreparedCall` (or a no-op for N = 0)."""
    _require_device(k, v, cos, sin, k_cache, v_cache, slot_mapping)
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous [num_blocks, Hkv, block_size, D] tensors of one shape")
    nb, hkv, bs, d = k_cache.shape
    if d % 2:
        raise ValueError(f"rotary embedding needs an even head_dim, got {d}")
    if k.dim() != 3 or k.shape != v.shape or k.shape[1:] != (hkv, d):
        raise ValueError(f"k/v must be [N, {hkv}, {d}], got {tuple(k.shape)} and {tuple(v.shape)}")
    n = k.shape[0]
    if q is not None:
        _require_device(q)
        if q.dim() != 3 or q.shape[0] != n or q.shape[2] != d or q.stride(2) != 1:
            raise ValueError(f"q must be [{n}, Hq, {d}] with a contiguous last dimension, got {tuple(q.shape)}")
    if cos.shape != (n, d) or sin.shape != (n, d) or cos.stride() != sin.stride() or cos.stride(1) != 1:
        raise ValueError(f"cos/sin must be [{n}, {d}] with one stride and a contiguous last dimension")
    dt = k_cache.dtype
    if any(t.dtype != dt for t in (k, v, cos, sin, v_cache) + ((q,) if q is not None else ())):
        raise TypeError("q, k, v, cos, sin and the cache must share one dtype")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("the last (head_dim) dimension of k/v must be contiguous")
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.shape[0] != n:
        raise ValueError("slot_mapping must be int64 [N]")
    if not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous")
    if n == 0:
        return _noop
    lib = _native.load()
    hq = 0 if q is None else q.shape[1]
    qp, qs0, qs1 = (None, 0, 0) if q is None else (q.data_ptr(), q.stride(0), q.stride(1))
    # Positions of the per-call addresses are _ROPE_SLOTS (q, k, v, cos, sin, k_cache, v_cache).
    args = (qp, qs0, qs1, k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), nb,
            slot_mapping.data_ptr(), n, hq, hkv, d, bs, dtype_code(dt), _stream_ptr(k_cache.device))
    return PreparedCall(lib.mip_rope_kv_append, args, "mip_rope_kv_append",
                        (q, k, v, cos, sin, k_cache, v_cache, slot_mapping))


_ROPE_SLOTS = (0, 3, 6, 9, 10, 12, 13)


def rope_kv_append(q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Rotate q and k in place (rotary embedding) and append the rotated k and v to the pool.

    ``q``: ``[N, Hq, D]`` (or None), ``k``/``v``: ``[N, Hkv, D]``, any token/head strides and a
    contiguous last dimension; ``cos``/``sin``: ``[N, D]`` rows per token. The values equal
    engine/model.py:216-224 (``x * cos + rotate_half(x) * sin`` evaluated op by op in the
    dtype) bit for bit, and the pool rows equal :func:`kv_append` of the rotated k and v.
    """
    prepare_rope_kv_append(q, k, v, cos, sin, k_cache, v_cache, slot_mapping)()


class _Workspace:
    """One scratch buffer per device, grown on demand (no initialisation needed).

    Calls that use it must be ordered (one stream, or graph replays on that stream): two
    decode calls running concurrently on different streams of one device would race on
    it; pass ``workspace=`` to each instead. A buffer that has been handed out is never
    freed: a captured graph may hold its address, so growing the workspace keeps the old
    buffer alive (``retired``) for the life of the process.
    """

    def __init__(self) -> None:
        self._bufs: dict[int, torch.Tensor] = {}
        self.retired: list[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        key = device.index if device.index is not None else torch.cuda.current_device()
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self.retired.append(buf)
            size = max(nbytes, 2 * buf.numel() if buf is not None else 0)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_workspace = _Workspace()


def decode_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                           max_blocks: int, dtype: torch.dtype) -> int:
    """Bytes of scratch a decode call of this shape needs (``mip_paged_decode_workspace``)."""
    return int(_native.load().mip_paged_decode_workspace(batch, num_heads, num_kv_heads, head_dim, block_size,
                                                         max_blocks, dtype_code(dtype)))


def _plan_key(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, block_size: int, max_blocks: int,
              dtype: torch.dtype) -> tuple:
    """The shape a work plan is laid out for (its tensor carries it as ``_mip_plan_key``)."""
    return (batch, num_heads, num_kv_heads, head_dim, block_size, max_blocks, dtype)


def prepare_paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                         context_lens: torch.Tensor, scale: float | None = None, out: torch.Tensor | None = None,
                         max_blocks: int | None = None, workspace: torch.Tensor | None = None,
                         append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
                         plan: torch.Tensor | None = None):
    """Validate a :func:`paged_decode` call once; returns ``(PreparedCall, out)``.

    ``append = (k, v, slot_mapping)`` prepares the fused append + decode call
    (:func:`paged_decode_append`) instead. ``plan`` is a work plan from :func:`decode_plan`
    for the same context lengths and block tables (or None).
    """
    _require_device(q, k_cache, v_cache, block_tables, context_lens)
    if q.dim() != 3 or q.stride(2) != 1:
        raise ValueError("q must be [B, Hq, D] with a contiguous last dimension")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous [num_blocks, Hkv, block_size, D] tensors of one shape")
    nb, hkv, bs, d = k_cache.shape
    b, hq, dq = q.shape
    if dq != d or hq % hkv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match the cache (Hkv={hkv}, D={d})")
    if q.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError("q and the cache must share one dtype")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise ValueError("block_tables must be int32 [B, max_blocks]")
    if block_tables.stride(1) != 1:
        raise ValueError("block_tables rows must be contiguous")
    if context_lens.dtype != torch.int32 or context_lens.shape != (b,) or not context_lens.is_contiguous():
        raise ValueError("context_lens must be contiguous int32 [B]")
    mb = block_tables.shape[1] if max_blocks is None else int(max_blocks)
    if mb < 1 or mb > block_tables.shape[1]:
        raise ValueError(f"max_blocks={mb} is outside [1, {block_tables.shape[1]}]")
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=q.device)
    elif out.shape != (b, hq, d) or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must be [B, Hq, D] in q's dtype with a contiguous last dimension")
    if b == 0:
        return _noop, out
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    code = dtype_code(q.dtype)
    lib = _native.load()
    need = int(lib.mip_paged_decode_workspace(b, hq, hkv, d, bs, mb, code))
    if workspace is None:
        workspace = _workspace.get(q.device, need)
    elif need and workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, needs {need}")
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    if plan is not None:
        _require_device(plan)
        if plan.dtype != torch.int32 or not plan.is_contiguous():
            raise ValueError("plan must be a contiguous int32 tensor from decode_plan")
        made_for = getattr(plan, "_mip_plan_key", None)
        want = _plan_key(b, hq, hkv, d, bs, mb, q.dtype)
        if made_for is not None and made_for != want:
            raise ValueError(f"the plan was made for shape {made_for}, not this call's {want}")
    plan_ptr = plan.data_ptr() if plan is not None else None
    plan_bytes = plan.numel() * 4 if plan is not None else 0
    # Positions of the per-call addresses are _DECODE_SLOTS (out, q, k_cache, v_cache), and
    # _APPEND_SLOTS (k, v, out, q, k_cache, v_cache) in the fused tuple below.
    args = (out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), nb, block_tables.data_ptr(), block_tables.stride(0),
            context_lens.data_ptr(), b, hq, hkv, d, bs, mb, scale, ws_ptr, ws_bytes, plan_ptr, plan_bytes, code,
            _stream_ptr(q.device))
    keep = (out, q, k_cache, v_cache, block_tables, context_lens, workspace, plan)
    if append is None:
        return PreparedCall(lib.mip_paged_decode, args, "mip_paged_decode", keep), out
    k, v, slot_mapping = append
    _require_device(k, v, slot_mapping)
    if k.shape != (b, hkv, d) or v.shape != (b, hkv, d):
        raise ValueError(f"k/v must be [{b}, {hkv}, {d}], got {tuple(k.shape)} and {tuple(v.shape)}")
    if k.dtype != k_cache.dtype or v.dtype != k_cache.dtype:
        raise TypeError("k, v and the cache must share one dtype")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("the last (head_dim) dimension of k/v must be contiguous")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (b,) or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous int64 [B]")
    fused = (k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1), slot_mapping.data_ptr(),
             *args)
    return PreparedCall(lib.mip_paged_decode_append, fused, "mip_paged_decode_append", keep + (k, v, slot_mapping)), out


_DECODE_SLOTS = (0, 3, 6, 7)
_APPEND_SLOTS = (0, 1, 7, 10, 13, 14)


def _layout(t: torch.Tensor) -> tuple:
    return (t.shape, t.stride(), t.dtype, t.device)


class DecodeStepCalls:
    """The per-layer calls of one decode step, with the step's fixed arguments checked once.

    Within a step every layer's call takes the same block tables, context lengths, slot
    mapping, plan and workspace; only q, k, v, the layer's pool and the output change, and
    they keep one layout. Each method runs the full checks of :func:`prepare_paged_decode` /
    :func:`prepare_rope_kv_append` when the layout of its tensors (shapes, strides, dtypes,
    devices) differs from the call before, and otherwise issues the same C-ABI call with
    the new addresses and the current stream. ``plan`` maps (num_heads, dtype) to the step's
    work plan (or None).
    """

    def __init__(self, block_tables: torch.Tensor, context_lens: torch.Tensor, slot_mapping: torch.Tensor,
                 scale: float, max_blocks: int, plan) -> None:
        self.block_tables, self.context_lens, self.slot_mapping = block_tables, context_lens, slot_mapping
        self.scale, self.max_blocks, self._plan = scale, max_blocks, plan
        self._cached: dict[str, tuple] = {}  # kind -> (layout key, fn, argument list, kept tensors)

    def _issue(self, kind: str, key: tuple, prepare, ptrs: tuple, slots: tuple, device: torch.device) -> None:
        hit = self._cached.get(kind)
        if hit is None or hit[0] != key:
            call = prepare()
            if call is _noop:
                return
            self._cached[kind] = (key, call._fn, list(call._args), call.keep)
            call()
            return
        _, fn, args, _ = hit
        for i, p in zip(slots, ptrs):
            args[i] = p
        args[-1] = _stream_ptr(device)
        st = fn(*args)
        if st:
            _native.check(st, fn.__name__)

    def decode_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor) -> torch.Tensor:
        """:func:`paged_decode_append` of one layer; returns ``out [B, Hq, D]``."""
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        key = (_layout(q), _layout(k), _layout(v), _layout(k_cache), _layout(v_cache))

        def prepare():
            return prepare_paged_decode(q, k_cache, v_cache, self.block_tables, self.context_lens, self.scale, out,
                                        self.max_blocks, append=(k, v, self.slot_mapping),
                                        plan=self._plan(q.shape[1], q.dtype))[0]

        self._issue("append", key, prepare, (k.data_ptr(), v.data_ptr(), out.data_ptr(), q.data_ptr(),
                                             k_cache.data_ptr(), v_cache.data_ptr()), _APPEND_SLOTS, q.device)
        return out

    def decode(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> torch.Tensor:
        """:func:`paged_decode` of one layer; returns ``out [B, Hq, D]``."""
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        key = (_layout(q), _layout(k_cache), _layout(v_cache))

        def prepare():
            return prepare_paged_decode(q, k_cache, v_cache, self.block_tables, self.context_lens, self.scale, out,
                                        self.max_blocks, plan=self._plan(q.shape[1], q.dtype))[0]

        self._issue("decode", key, prepare, (out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()),
                    _DECODE_SLOTS, q.device)
        return out

    def rope_append(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
        """:func:`rope_kv_append` of one layer (q and k rotated in place)."""
        key = (_layout(q), _layout(k), _layout(v), _layout(cos), _layout(sin), _layout(k_cache), _layout(v_cache))

        def prepare():
            return prepare_rope_kv_append(q, k, v, cos, sin, k_cache, v_cache, self.slot_mapping)

        self._issue("rope", key, prepare, (q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                           k_cache.data_ptr(), v_cache.data_ptr()), _ROPE_SLOTS, k.device)


def prepare_decode_plan(context_lens: torch.Tensor, block_tables: torch.Tensor, num_heads: int, num_kv_heads: int,
                        head_dim: int, block_size: int, dtype: torch.dtype, max_blocks: int | None = None,
                        plan: torch.Tensor | None = None):
    """A prepared :func:`decode_plan` launch and its plan tensor, or ``(None, None)`` where the
    stream kernel does not run (then decode calls take no plan)."""
    _require_device(context_lens, block_tables)
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be int32 [B, max_blocks] with contiguous rows")
    b = block_tables.shape[0]
    if context_lens.dtype != torch.int32 or context_lens.shape != (b,) or not context_lens.is_contiguous():
        raise ValueError("context_lens must be contiguous int32 [B]")
    mb = block_tables.shape[1] if max_blocks is None else int(max_blocks)
    code = dtype_code(dtype)
    lib = _native.load()
    need = int(lib.mip_paged_decode_plan_bytes(b, num_heads, num_kv_heads, head_dim, block_size, mb, code))
    if need == 0:
        return None, None
    if plan is None:
        plan = torch.empty(-(-need // 4), dtype=torch.int32, device=context_lens.device)
    elif plan.dtype != torch.int32 or not plan.is_contiguous() or plan.numel() * 4 < need:
        raise ValueError(f"plan must be a contiguous int32 tensor of at least {need} bytes")
    plan._mip_plan_key = _plan_key(b, num_heads, num_kv_heads, head_dim, block_size, mb, dtype)
    args = (context_lens.data_ptr(), block_tables.data_ptr(), block_tables.stride(0), b, num_heads, num_kv_heads,
            head_dim, block_size, mb, code, plan.data_ptr(), plan.numel() * 4, _stream_ptr(context_lens.device))
    keep = (context_lens, block_tables, plan)
    return PreparedCall(lib.mip_paged_decode_plan, args, "mip_paged_decode_plan", keep), plan


def decode_plan(context_lens: torch.Tensor, block_tables: torch.Tensor, num_heads: int, num_kv_heads: int,
                head_dim: int, block_size: int, dtype: torch.dtype, max_blocks: int | None = None,
                plan: torch.Tensor | None = None) -> torch.Tensor | None:
    """One decode step's work plan for the stream kernel (None where that kernel does not run).

    Every layer's :func:`paged_decode` / :func:`paged_decode_append` with these context
    lengths and tables can take it and skip deriving the work split.
    """
    call, plan = prepare_decode_plan(context_lens, block_tables, num_heads, num_kv_heads, head_dim, block_size,
                                     dtype, max_blocks, plan)
    if call is not None:
        call()
    return plan


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor, scale: float | None = None, out: torch.Tensor | None = None,
                 max_blocks: int | None = None, workspace: torch.Tensor | None = None,
                 plan: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention over paged K/V for one query token per sequence.

    ``q``: ``[B, Hq, D]`` (last dim contiguous). ``k_cache``/``v_cache``: one layer,
    ``[num_blocks + 1, Hkv, block_size, D]``. ``block_tables``: int32 ``[B, >= max_blocks]``.
    ``context_lens``: int32 ``[B]`` (keys attended = positions + 1). Returns ``out``
    ``[B, Hq, D]`` in q's dtype. Follows engine/kv_cache.py:615-620 and
    engine/model.py:126-147 with ``scale = 1/sqrt(D)`` by default.
    """
    call, out = prepare_paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale, out, max_blocks,
                                     workspace, plan=plan)
    call()
    return out


def prepare_paged_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                          cu_q: torch.Tensor, ctx_start: torch.Tensor, max_q_len: int, scale: float | None = None,
                          out: torch.Tensor | None = None, max_blocks: int | None = None):
    """Validate a :func:`paged_prefill` call once; returns ``(PreparedCall, out)``."""
    _require_device(q, k_cache, v_cache, block_tables, cu_q, ctx_start)
    if q.dim() != 3 or q.stride(2) != 1:
        raise ValueError("q must be [N, Hq, D] with a contiguous last dimension")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous [num_blocks, Hkv, block_size, D] tensors of one shape")
    nb1, hkv, bs, d = k_cache.shape
    n, hq, dq = q.shape
    if dq != d or hq % hkv:
        raise ValueError(f"q {tuple(q.shape)} does not match the pool (Hkv={hkv}, D={d})")
    if q.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise TypeError("q and the cache must share one dtype")
    if block_tables.dtype != torch.int32 or cu_q.dtype != torch.int32 or ctx_start.dtype != torch.int32:
        raise TypeError("block_tables, cu_q and ctx_start must be int32")
    num_seqs = ctx_start.shape[0]
    if block_tables.dim() != 2 or block_tables.shape[0] < num_seqs or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be [S, nb] with contiguous rows")
    if cu_q.shape != (num_seqs + 1,) or not (cu_q.is_contiguous() and ctx_start.is_contiguous()):
        raise ValueError("cu_q must be int32 [S + 1] and ctx_start int32 [S], contiguous")
    nbm = block_tables.shape[1] if max_blocks is None else max_blocks
    if out is None:
        out = torch.empty(n, hq, d, dtype=q.dtype, device=q.device)
    elif out.shape != (n, hq, d) or out.dtype != q.dtype or out.stride(2) != 1:
        raise ValueError("out must be [N, Hq, D] in q's dtype with a contiguous last dimension")
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    lib = _native.load()
    args = (out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(),
            v_cache.data_ptr(), nb1, block_tables.data_ptr(), block_tables.stride(0), cu_q.data_ptr(),
            ctx_start.data_ptr(), num_seqs, max_q_len, hq, hkv, d, bs, nbm, scale, dtype_code(q.dtype),
            _stream_ptr(q.device))
    keep = (out, q, k_cache, v_cache, block_tables, cu_q, ctx_start)
    return PreparedCall(lib.mip_paged_prefill, args, "mip_paged_prefill", keep), out


def paged_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                  cu_q: torch.Tensor, ctx_start: torch.Tensor, max_q_len: int, scale: float | None = None,
                  out: torch.Tensor | None = None, max_blocks: int | None = None) -> torch.Tensor:
    """Varlen causal attention of packed new tokens over their sequences' paged keys.

    ``q``: ``[N, Hq, D]`` packed rows (last dim contiguous); sequence ``s`` owns rows
    ``cu_q[s] .. cu_q[s+1]-1`` (int32 ``[S+1]``), at positions ``ctx_start[s] + i``
    (int32 ``[S]``), and each row attends its sequence's keys ``0 .. position`` read from the
    pool through ``block_tables`` (int32 ``[S, >= max_blocks]``). Returns ``out [N, Hq, D]``.
    Follows engine/kv_cache.py:268-294 (prefix read-back + mask) and :290-294 (packed causal).
    16-bit data at head_dim 64/128 runs the MFMA prefill kernel, other shapes (fp32, other
    head sizes, at most 8 query heads per kv head) the VALU kernel; anything else raises.
    """
    call, out = prepare_paged_prefill(q, k_cache, v_cache, block_tables, cu_q, ctx_start, max_q_len, scale, out,
                                      max_blocks)
    call()
    return out


def paged_decode_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                        v_cache: torch.Tensor, slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                        context_lens: torch.Tensor, scale: float | None = None, out: torch.Tensor | None = None,
                        max_blocks: int | None = None, workspace: torch.Tensor | None = None,
                        plan: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`kv_append` of the step's ``k``/``v`` ``[B, Hkv, D]`` at ``slot_mapping``, then
    :func:`paged_decode`, as one call (engine/kv_cache.py:611-620). One kernel launch on the
    stream-kernel path; ``slot_mapping[b]`` must be the slot of key ``context_lens[b] - 1``
    (or outside the pool).
    """
    call, out = prepare_paged_decode(q, k_cache, v_cache, block_tables, context_lens, scale, out, max_blocks,
                                     workspace, append=(k, v, slot_mapping), plan=plan)
    call()
    return out


def _copy_shape(k_pool: torch.Tensor, v_pool: torch.Tensor) -> tuple[int, int, int]:
    if k_pool.shape != v_pool.shape or k_pool.dim() != 5 or not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("k_pool/v_pool must be contiguous [L, num_blocks, Hkv, block_size, D] tensors of one shape")
    return k_pool.shape[0], k_pool.shape[1], k_pool[0, 0].numel() * k_pool.element_size()


def _host_pairs(pairs) -> np.ndarray:
    """A private contiguous int64 [n, 2] copy of ``pairs`` (a CPU tensor, an array or a
    sequence of (src, dst)), so a prepared call keeps the pairs it was prepared with."""
    if isinstance(pairs, torch.Tensor):
        pairs = pairs.numpy()
    return np.array(pairs, dtype=np.int64, copy=True, order="C").reshape(-1, 2)


def prepare_copy_blocks(k_pool: torch.Tensor, v_pool: torch.Tensor, pairs):
    """Validate a :func:`copy_blocks` call once; returns a :class:`PreparedCall` (or a no-op for no pairs).

    ``pairs`` on the pool's device: ``mip_copy_blocks`` reads them from device memory (a
    graph replay sees later writes to that tensor). Anything else (a CPU tensor, an array, a
    sequence of (src, dst)): ``mip_copy_blocks_host`` passes them in the kernel arguments, as
    they are when the call is prepared.
    """
    _require_device(k_pool, v_pool)
    num_layers, nb, block_bytes = _copy_shape(k_pool, v_pool)
    stream = _stream_ptr(k_pool.device)
    if isinstance(pairs, torch.Tensor) and pairs.is_cuda:
        _require_device(pairs)
        if pairs.dtype != torch.int64 or pairs.dim() != 2 or pairs.shape[1] != 2 or not pairs.is_contiguous():
            raise ValueError("pairs must be contiguous int64 [n, 2]")
        if pairs.device != k_pool.device:
            raise ValueError("pairs on a device must be on the pool's device")
        n = pairs.shape[0]
        if n == 0:
            return _noop
        args = (k_pool.data_ptr(), v_pool.data_ptr(), pairs.data_ptr(), n, num_layers, nb, block_bytes, stream)
        return PreparedCall(_native.load().mip_copy_blocks, args, "mip_copy_blocks", (k_pool, v_pool, pairs))
    arr = _host_pairs(pairs)
    n = arr.shape[0]
    if n == 0:
        return _noop
    args = (k_pool.data_ptr(), v_pool.data_ptr(), arr.ctypes.data, n, num_layers, nb, block_bytes, stream)
    return PreparedCall(_native.load().mip_copy_blocks_host, args, "mip_copy_blocks_host", (k_pool, v_pool, arr))


def copy_blocks(k_pool: torch.Tensor, v_pool: torch.Tensor, pairs) -> None:
    """Copy whole blocks, every layer, K and V: ``pool[:, dst] = pool[:, src]`` per (src, dst) row.

    ``k_pool``/``v_pool``: ``[num_layers, num_blocks + 1, Hkv, block_size, D]`` contiguous.
    ``pairs``: int64 ``[n, 2]`` on the pool's device, or (src, dst) pairs on the host (a CPU
    tensor, an array or a sequence), which travel in the kernel arguments with no upload.
    Bitwise copy (no reference counterpart; used for copy-on-write of shared prefix blocks).
    """
    prepare_copy_blocks(k_pool, v_pool, pairs)()
