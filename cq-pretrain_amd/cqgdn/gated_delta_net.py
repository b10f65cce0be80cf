"""MI355X GDN training/inference backend (``gdn_backend: hip``), no eager fallback.

Host-side mirror of the reference's ``ops/gated_delta_net.py``: the same public
functions (``initialize``, ``call``, ``CALLS``, ``host_bounds``, ``chunk_indices``,
``device_metadata``, ``reverse_cumsum``, ``delta``, ``prefill``, ``recurrent``,
``gated_norm``, ``conv``, ``provenance``) with the same argument meaning, layouts
and error behaviour.  The device work runs in hand-written gfx950 HIP kernels of
``libcqgdn.so`` (C ABI in include/cqgdn.h), enqueued on the current stream.  Two
modes, as the reference's (``DELTA_HIP_MODE``, read at import like
``DELTA_ASCENDC_MODE``, ops/gated_delta_net.py:20): ``cached`` (the default here) keeps
the forward's workspace (w, h, v_new and the rest) for the backward, so the serial
state scan runs once; ``fused`` keeps only the inputs between the forward and the
backward, which rebuilds the workspace (chunk preparation and state scan again)
before it runs, trading that time for the workspace's memory across layers.

PyTorch only supplies device memory and streams.  Every contract violation raises
``ValueError``/``NotImplementedError`` before any launch, like the reference.
"""

from __future__ import annotations

import ctypes
import os
from collections import Counter
from functools import lru_cache

import torch

from . import _lib

CALLS = Counter()
MODE = os.getenv("DELTA_HIP_MODE", "cached")
CHUNK = 64
_INITIALIZED = False


def initialize():
    """Load libcqgdn and check the device and the mode (ops/gated_delta_net.py:24-59)."""
    global _INITIALIZED
    if MODE not in ("fused", "cached"):
        raise ValueError(f"Unknown DELTA_HIP_MODE={MODE}")
    _lib.lib()
    if torch.cuda.is_available():
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
        if not arch.startswith("gfx950"):
            raise RuntimeError(f"libcqgdn is built for gfx950, the current device is {arch}")
    _INITIALIZED = True


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t):
    # a plain int: the C-ABI signatures declare c_void_p, which ctypes converts from int
    return t.data_ptr() if t is not None else None


def call(name, *args):
    """Invoke one C-ABI entry point, counting calls per op (ops/gated_delta_net.py:62-64)."""
    CALLS[name] += 1
    _lib.check(getattr(_lib.lib(), name)(*args), name)


def _rows_view(t, rows, width):
    """``t`` as [rows, width] with unit channel stride and a constant row stride, without a
    copy when ``t`` is such a view already (a column slice of a wider projection)."""
    try:
        v = t.view(rows, width)
    except RuntimeError:
        v = t.reshape(rows, width)
    if v.stride(1) != 1 or v.stride(0) % 8 or v.data_ptr() % 16:
        v = v.contiguous()
    return v


class _GatedNorm(torch.autograd.Function):
    """Gated RMSNorm over D = 128 with an optional fused row gather, on the GPU."""

    @staticmethod
    def forward(ctx, y, z, weight, eps, index, zero_rows):
        H = y.shape[-2]
        yc = y.contiguous()
        rows = index.numel() if index is not None else yc.numel() // (H * 128)
        zv = _rows_view(z, rows, H * 128)
        w = weight.float().contiguous()
        out = torch.empty(rows, H, 128, dtype=y.dtype, device=y.device)
        rstd = torch.empty(rows, H, dtype=torch.float32, device=y.device)
        call("cqgdn_gated_norm_fwd", _ptr(yc), _ptr(index), rows, H, _ptr(zv), zv.stride(0), _ptr(w), float(eps),
             _ptr(out), _ptr(rstd), _stream(y.device))
        ctx.save_for_backward(yc, zv, w, rstd, index, zero_rows)
        ctx.shapes, ctx.wdtype = (y.shape, z.shape), weight.dtype
        return out if index is not None else out.reshape(y.shape)

    @staticmethod
    def backward(ctx, dout):
        yc, zv, w, rstd, index, zero_rows = ctx.saved_tensors
        rows, H = rstd.shape
        do = dout.contiguous()
        dy = torch.empty_like(yc)
        dz = torch.empty(rows, H * 128, dtype=zv.dtype, device=zv.device)
        dw = torch.empty(128, dtype=torch.float32, device=zv.device)
        ws = torch.empty(max(_lib.lib().cqgdn_gated_norm_bwd_workspace_size(rows, H), 16), dtype=torch.uint8,
                         device=zv.device)
        n_zero = zero_rows.numel() if zero_rows is not None else 0
        call("cqgdn_gated_norm_bwd", _ptr(yc), _ptr(index), _ptr(zero_rows), n_zero, rows, H, _ptr(zv), zv.stride(0),
             _ptr(w), _ptr(rstd), _ptr(do), _ptr(dy), _ptr(dz), dz.stride(0), _ptr(dw), _ptr(ws), ws.numel(),
             _stream(zv.device))
        return dy.reshape(ctx.shapes[0]), dz.reshape(ctx.shapes[1]), dw.to(ctx.wdtype), None, None, None


def unread_rows(index, y_rows):
    """Device int32 list of the rows of y that ``index`` never reads (the rows the fused
    gated_norm backward writes with zeros); checks that ``index`` repeats no row."""
    real = index[index >= 0].long()
    counts = torch.bincount(real, minlength=y_rows)
    if counts.numel() > y_rows or (counts.numel() and int(counts.max()) > 1):
        raise ValueError("index must hold distinct values in [-1, len(y))")
    return (counts == 0).nonzero().flatten().to(torch.int32)


def gated_norm(y, z, weight, eps=1e-6, *, index=None, zero_rows=None):
    """RMSNorm(y) * weight * silu(z) over D = 128 (ops/gated_delta_net.py:67-74; CPU form
    models/backbone_qwen35.py:107-114), y and z bf16 [..., H, 128] on the GPU, computed in fp32.

    ``index`` (device int32 [rows], values in [-1, len(y))) fuses the layer's output gather
    (models/backbone_qwen35.py:242-246): row r normalizes y[index[r]], and a zero row for -1
    (a padding row); z is then [rows, H, 128] and may be a column slice of the fused
    projection.  ``zero_rows`` (from ``unread_rows``, cached per plan by callers) lists the y
    rows no r reads; it is derived here when omitted.
    """
    if y.shape[-1] != 128 or y.dim() < 2:
        raise ValueError("gated_norm expects y [..., H, 128]")
    if y.dtype != torch.bfloat16 or z.dtype != torch.bfloat16:
        raise NotImplementedError("the hip gated_norm kernels compute on bf16 y and z")
    if weight.shape != (128,):
        raise ValueError("weight must be [128]")
    _require_gpu(y, z, weight)
    if index is None:
        if z.shape != y.shape:
            raise ValueError("y and z must have the same shape")
    else:
        if y.dim() != 3 or index.dim() != 1 or z.shape != (index.numel(), y.shape[1], 128):
            raise ValueError("with index, y is [y_rows, H, 128], index [rows] and z [rows, H, 128]")
        index = index.to(torch.int32)
        if zero_rows is None:
            zero_rows = unread_rows(index, y.shape[0])
    return _GatedNorm.apply(y, z, weight, eps, index, zero_rows)


def _require_gpu(*tensors):
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("the hip GDN backend requires tensors on a ROCm GPU")


def reverse_cumsum(dg, bounds):
    """Reverse chunk-local cumsum (chunk 64) of dg in the reference's head-first layout [B,H,T]
    (ops/gated_delta_net.py:77-87, called at :204 on the backward's head-first dg), fp32 out.

    Packed bounds (B == 1) restart the chunks at every document; without bounds every batch
    row is its own sequence."""
    _require_gpu(dg)
    b, h, t = dg.shape
    x = dg.transpose(1, 2).reshape(b * t, h).float().contiguous()  # the kernel's time-first rows
    bounds = tuple(range(0, b * t + 1, t)) if bounds is None else bounds
    if bounds[-1] != b * t:
        raise ValueError("bounds must cover every token")
    _, table, _ = device_metadata(bounds, str(dg.device))
    out = torch.empty_like(x)
    call("cqgdn_chunk_local_cumsum", _ptr(x), _ptr(out), b * t, h, _ptr(table), table.shape[0], 1,
         _stream(dg.device))
    return out.reshape(b, t, h).transpose(1, 2).contiguous()


@lru_cache(maxsize=128)
def chunk_indices(bounds, size):
    """Flat (document, chunk) pairs for chunk ``size`` (ops/gated_delta_net.py:90-99)."""
    if bounds is None:
        return None
    return [
        item
        for i, (a, b) in enumerate(zip(bounds, bounds[1:]))
        for j in range((b - a + size - 1) // size)
        for item in (i, j)
    ]


def host_bounds(cu_seqlens, cu_seqlens_cpu):
    """Host copy of packed-sequence bounds; never reads device metadata (ops/gated_delta_net.py:102-114)."""
    if cu_seqlens is None:
        return None
    if cu_seqlens_cpu is None:
        raise ValueError("Supply cu_seqlens_cpu: training must not copy metadata from the GPU in each layer")
    if isinstance(cu_seqlens_cpu, torch.Tensor):
        if cu_seqlens_cpu.device.type != "cpu":
            raise ValueError("cu_seqlens_cpu must be on CPU")
        cu_seqlens_cpu = cu_seqlens_cpu.tolist()
    bounds = tuple(int(i) for i in cu_seqlens_cpu)
    if not bounds or bounds[0] != 0 or any(b < a for a, b in zip(bounds, bounds[1:])):
        raise ValueError("Invalid packed sequence boundaries")
    return bounds


def chunk_table(bounds):
    """Host (CPU int32) chunk table [n_chunks, 2] = (start, len) and doc_chunk [n_docs + 1]."""
    n_bounds = len(bounds)
    b = (ctypes.c_int64 * n_bounds)(*bounds)
    n = _lib.lib().cqgdn_chunk_table(b, n_bounds, None, None)
    if n < 0:
        raise ValueError(_lib.lib().cqgdn_last_error().decode())
    table = torch.empty(max(n, 1), 2, dtype=torch.int32)
    doc = torch.empty(n_bounds, dtype=torch.int32)
    _lib.lib().cqgdn_chunk_table(b, n_bounds, ctypes.c_void_p(table.data_ptr()), ctypes.c_void_p(doc.data_ptr()))
    return table[:n], doc


@lru_cache(maxsize=64)
def device_metadata(bounds, device):
    """Device copies of the bounds and chunk tables, cached per bounds (ops/gated_delta_net.py:117-126).

    Returns ``(cu int64 [n_docs+1], chunk_table int32 [n_chunks,2], doc_chunk int32 [n_docs+1])``.
    """
    if bounds is None:
        return None, None, None
    table, doc = chunk_table(bounds)
    cu = torch.tensor(bounds, dtype=torch.long)
    return (cu.to(device, non_blocking=True), table.to(device, non_blocking=True),
            doc.to(device, non_blocking=True))


def _as(x, dtype):
    """x contiguous in ``dtype``; x itself when it already is (no torch call on the hot path)."""
    return x if x.dtype == dtype and x.is_contiguous() else x.to(dtype).contiguous()


def _flatten(q, k, v, g, beta, bounds):
    """Packed [1,T,...] views; unpacked batches become one document per row.  q, k, v keep their
    dtype, bf16 or fp16 (one for all three): the kernels compute with operands of that type."""
    b, t = q.shape[0], q.shape[1]
    if bounds is None:
        bounds = tuple(range(0, b * t + 1, t)) if t > 0 else (0,) * (b + 1)
    if b != 1:
        q, k, v, g, beta = (x.reshape(1, b * t, *x.shape[2:]) for x in (q, k, v, g, beta))
    dt = q.dtype if q.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    q, k, v = (_as(x, dt) for x in (q, k, v))
    g, beta = (_as(x, torch.float32) for x in (g, beta))
    return q, k, v, g, beta, bounds


def _forward(q, k, v, g, beta, bounds, normalize, scale, training, initial_state=None, want_state=False,
             precise=False, output=True):
    t, h = q.shape[1], q.shape[2]
    if q.shape[0] != 1 or bounds[0] != 0 or bounds[-1] != t:
        raise ValueError("packed forward needs batch 1 and bounds (0, ..., T) covering every event")
    for x in (q, k, v, g, beta):
        if not x.is_contiguous():
            raise ValueError("forward operands must be contiguous")
    if initial_state is not None and initial_state.shape != (len(bounds) - 1, h, 128, 128):
        raise ValueError("initial_state must be [n_docs, H, 128, 128] fp32")
    cu, table, doc = device_metadata(bounds, str(q.device))
    flags = (_lib.NORMALIZE if normalize else 0) | (_lib.TRAINING if training else 0) | \
        (_lib.PRECISE if precise else 0) | (0 if output else _lib.NO_OUTPUT)
    CALLS["cqgdn_fwd"] += 1
    o, state, ws = _lib.ops().fwd(q, k, v, g, beta, table, doc, float(scale), flags, initial_state, want_state)
    o = o if output else None
    state = state if want_state else None
    return o, state, ws


class _Delta(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, g, beta, bounds, normalize, scale):
        ctx.input_dtypes = [x.dtype for x in (q, k, v, g, beta)]
        ctx.shapes = [x.shape for x in (q, k, v, g, beta)]
        qf, kf, vf, gf, bf, bounds = _flatten(q, k, v, g, beta, bounds)
        o, _, ws = _forward(qf, kf, vf, gf, bf, bounds, normalize, scale, training=True)
        ctx.mode = MODE
        if MODE == "fused":  # the inputs only: the backward rebuilds the workspace
            ctx.save_for_backward(qf, kf, vf, gf, bf)
        else:
            ctx.save_for_backward(qf, kf, vf, gf, bf, ws)
        ctx.bounds, ctx.scale, ctx.normalize = bounds, scale, normalize
        return o if o.shape == v.shape and o.dtype == v.dtype else o.reshape(v.shape).to(v.dtype)

    @staticmethod
    def backward(ctx, dy):
        if ctx.mode == "fused":  # one call rebuilds the forward workspace and runs the backward
            q, k, v, g, beta = ctx.saved_tensors
            grads = _backward(q, k, v, g, beta, None, dy, ctx.bounds, ctx.normalize, ctx.scale)
        else:
            q, k, v, g, beta, ws = ctx.saved_tensors
            grads = _backward(q, k, v, g, beta, ws, dy, ctx.bounds, ctx.normalize, ctx.scale)
        grads = [x if x.shape == shape and x.dtype == dtype else x.reshape(shape).to(dtype)
                 for x, shape, dtype in zip(grads, ctx.shapes, ctx.input_dtypes)]
        return *grads, None, None, None


def _backward(q, k, v, g, beta, ws, dy, bounds, normalize, scale):
    """dq, dk, dv, dg, dbeta of the packed chunked forward whose TRAINING workspace is ``ws``; with
    ``ws`` None the workspace is rebuilt inside the same call (fused mode)."""
    cu, table, doc = device_metadata(bounds, str(v.device))
    if dy.shape != v.shape:
        dy = dy.reshape(v.shape)
    dy = _as(dy, v.dtype)
    flags = (_lib.NORMALIZE if normalize else 0) | _lib.TRAINING
    CALLS["cqgdn_bwd" if ws is not None else "cqgdn_bwd_recompute"] += 1
    dq, dk, dv, dg, db = _lib.ops().bwd(q, k, v, g, beta, dy, table, doc, float(scale), flags, ws)
    return dq, dk, dv, dg, db


def delta(
    q,
    k,
    v,
    g,
    beta,
    *,
    use_qk_l2norm_in_kernel=False,
    cu_seqlens=None,
    cu_seqlens_cpu=None,
    initial_state=None,
    output_final_state=False,
    scale=None,
):
    """Chunked GDN for training, same contract as ops/gated_delta_net.py:217-249.

    q, k, v: [B,T,H,128] bf16 or fp16 time-first; g, beta: [B,T,H] (computed in fp32).
    Packed documents: B == 1 with ``cu_seqlens`` (device) and ``cu_seqlens_cpu``
    (host) bounds; the state resets at each document.  Returns ``(o, None)``, o and the
    gradients in the input dtypes.  The kernels' MFMA operands take the inputs' type: fp16
    inputs run the fp16 kernels (CQGDN_FP16), with V and dO scaled by powers of two inside the
    calls so that every fp16 operand stays in range.
    """
    if initial_state is not None or output_final_state:
        raise NotImplementedError("This training adapter requires zero initial state and no state output")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("QKV must share BF16/FP16 dtype")
    if q.shape != k.shape or q.shape != v.shape or (q.shape[-1] != 128 or q.shape[-2] not in (4, 8, 16, 32)):
        raise ValueError("GDN requires equal expanded QKV, head dimension 128 and supported local heads")
    bounds = host_bounds(cu_seqlens, cu_seqlens_cpu)
    if bounds is not None and (q.shape[0] != 1 or bounds[-1] != q.shape[1]):
        raise ValueError("Packed inputs must have batch 1 and boundaries covering every token")
    if g.shape != q.shape[:3] or beta.shape != q.shape[:3]:
        raise ValueError("g and beta must be [B,T,H]")
    _require_gpu(q, k, v, g, beta)
    return _Delta.apply(
        q,
        k,
        v,
        g,
        beta,
        bounds,
        use_qk_l2norm_in_kernel,
        q.shape[-1] ** -0.5 if scale is None else float(scale),
    ), None


@torch.no_grad()
def prefill(q, k, v, g, beta, bounds, initial_state=None):
    """Inference forward with per-document final states (ops/gated_delta_net.py:292-311).

    Runs the precise forward (fp16 MFMA operands, CQGDN_PRECISE), whose final states
    stay within 1e-3 relative of an fp32 computation.
    q, k, v: [1,T,H,128] bf16 or fp16 (l2norm applied inside, scale 128^-0.5); g, beta [1,T,H].
    fp16 inputs are read as fp16 (CQGDN_FP16), bf16 inputs are rounded to fp16 operands.
    Returns ``(o [1,T,H,128] time-first in the dtype of q, state [n_docs,H,K,V] fp32)``.
    """
    bounds = tuple(int(b) for b in bounds)
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("prefill needs bf16 or fp16 q/k/v")
    if q.shape[0] != 1 or bounds[0] != 0 or bounds[-1] != q.shape[1]:
        raise ValueError("prefill needs batch 1 and bounds covering every token")
    _require_gpu(q, k, v, g, beta)
    qf, kf, vf, gf, bf, bounds = _flatten(q, k, v, g, beta, bounds)
    if initial_state is not None:
        initial_state = initial_state.float().contiguous()
    o, state, _ = _forward(qf, kf, vf, gf, bf, bounds, True, q.shape[-1] ** -0.5, training=False,
                           initial_state=initial_state, want_state=True, precise=True)
    return _as(o, q.dtype), state


@torch.no_grad()
def recurrent(q, k, v, g, beta, state, out):
    """One recurrent decode pass over t events, state updated in place (ops/gated_delta_net.py:314-352).

    q, k (l2-normalized), v, out: [t,H,128], all bf16 or all fp16 (read and written as
    such; the arithmetic is fp32 either way); g: [t,H] fp32; beta: [t,H] fp32 or bf16;
    state: [1,H,V,K] fp32 value-first.  Batched decode passes q of shape [N,t,H,128],
    g/beta [N,t,H] and state [N,H,V,K].
    """
    # the contract checks (ValueError texts of the reference's adapter) run inside the operator
    CALLS["cqgdn_recurrent"] += 1
    _lib.ops().recurrent(q, k, v, g, beta, state, out, 128 ** -0.5)
    return out


def l2_fwd(x):
    """Row l2norm over the last dim 128; returns (y, rstd) (the reference's ``l2_fwd`` op)."""
    _require_gpu(x)
    if x.shape[-1] != 128 or x.dtype != torch.bfloat16:
        raise ValueError("l2_fwd needs bf16 rows of 128")
    x = x.contiguous()
    y = torch.empty_like(x)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    call("cqgdn_l2norm_fwd", _ptr(x), _ptr(y), _ptr(rstd), x.numel() // 128, _stream(x.device))
    return y, rstd


def l2_bwd(y, rstd, dy):
    """Backward of ``l2_fwd``: dx = rstd * (dy - y (y . dy))."""
    _require_gpu(y, rstd, dy)
    y, dy, rstd = y.contiguous(), dy.to(y.dtype).contiguous(), rstd.float().contiguous()
    dx = torch.empty_like(y)
    call("cqgdn_l2norm_bwd", _ptr(y), _ptr(rstd), _ptr(dy), _ptr(dx), y.numel() // 128, _stream(y.device))
    return dx


@lru_cache(maxsize=64)
def _conv_bounds(bounds, device):
    """Device int32 document bounds for the conv kernels, cached per bounds."""
    return torch.tensor(bounds, dtype=torch.int32).to(device, non_blocking=True)


class _Conv(torch.autograd.Function):
    """Packed depthwise causal conv1d on the GPU (ops/gated_delta_net.py:252-277): the forward
    saves only x and the weight; the backward recomputes the pre-activation in the kernel."""

    @staticmethod
    def forward(ctx, x, weight, activation, bounds):
        xf = x.contiguous().reshape(-1, x.shape[-1])
        w = weight.contiguous()
        cb = _conv_bounds(bounds, x.device)
        y = torch.empty_like(xf)
        call("cqgdn_conv1d_fwd", _ptr(xf), _ptr(w), _ptr(cb), len(bounds) - 1, xf.shape[0], xf.shape[1], w.shape[1],
             int(activation), _ptr(y), _stream(x.device))
        ctx.save_for_backward(xf, w)
        ctx.shape, ctx.bounds, ctx.activation = x.shape, bounds, activation
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        xf, w = ctx.saved_tensors
        dyf = dy.contiguous().reshape(xf.shape)
        T, C, K = xf.shape[0], xf.shape[1], w.shape[1]
        dx = torch.empty_like(xf)
        dw = torch.empty(C, K, dtype=torch.float32, device=xf.device)
        ws = torch.empty(_lib.lib().cqgdn_conv1d_bwd_workspace_size(T, C, K), dtype=torch.uint8, device=xf.device)
        cb = _conv_bounds(ctx.bounds, xf.device)
        call("cqgdn_conv1d_bwd", _ptr(xf), _ptr(w), _ptr(dyf), _ptr(cb), len(ctx.bounds) - 1, T, C, K,
             int(ctx.activation), _ptr(dx), _ptr(dw), _ptr(ws), ws.numel(), _stream(xf.device))
        return dx.reshape(ctx.shape), dw.to(w.dtype), None, None


def conv(x, weight, *, activation=None, cu_seqlens=None, cu_seqlens_cpu=None):
    """Packed causal conv1d, x [1,T,C] (or [B,T,C] unpacked), weight [C,K] (ops/gated_delta_net.py:280-289).

    Returns ``(y, None)`` like the reference; documents never see each other's rows.
    """
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"Unsupported activation {activation}")
    if weight.dim() != 2 or weight.shape[0] != x.shape[-1]:
        raise ValueError("weight must be [channels, kernel]")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise NotImplementedError("the hip conv kernels compute on bf16 x and weight")
    _require_gpu(x, weight)
    bounds = host_bounds(cu_seqlens, cu_seqlens_cpu)
    if bounds is None:  # unpacked: every batch row is its own document
        bounds = tuple(i * x.shape[1] for i in range(x.shape[0] + 1))
    elif x.shape[0] != 1 or bounds[-1] != x.shape[1]:
        raise ValueError("Packed inputs must have batch 1 and boundaries covering every token")
    return _Conv.apply(x, weight, activation is not None, bounds), None


def provenance():
    """Backend record: library hash and version, device, per-op call counts (ops/gated_delta_net.py:355-376)."""
    device = None
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        device = dict(name=props.name, arch=props.gcnArchName)
    return dict(
        backend="hip",
        mode=MODE,
        library=str(_lib.LIB_PATH),
        version=_lib.version(),
        sha256={_lib.LIB_PATH.name: _lib.sha256()},
        device=device,
        calls=dict(CALLS),
        fallback={},
    )
