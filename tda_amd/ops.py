"""Host side of the threshold-attention operator: tensor checks, buffer allocation, the C-ABI
calls and the autograd.Function.

Mirrors ThresholdRelaFunction of the reference (snap-research/TDA
triton_threshold_attention.py, TTA:327-469) with these differences:
  * one Function covers both the single-branch (TRA) and the fused two-branch (TDA) form;
  * beta and lambda are device tensors read by the kernels: no .item() sync (TTA:352);
  * inputs are neither up-cast nor copied (TTA:356-360); bf16 stays bf16 with fp32
    accumulation, fp32 stays fp32 (float16 and float64 are computed in fp32 and cast back,
    as the reference does for every dtype);
  * the backward also returns d beta and d lambda (the reference returns None, TTA:469);
  * the forward saves the inputs, the inverse row norms and a tile-occupancy bitmask instead
    of fp32 copies of q, k, v (TTA:396).

Per-call host cost.  A training step runs the forward and the backward of the op once per
layer, and both must be enqueued faster than the GPU runs them (about 0.33 ms at the headline
shape) or the GPU idles between steps.  So the argument structs of the C ABI are built once
per configuration (shapes, strides, dtype, flags) and cached as byte templates: a call copies
the template and writes only the device pointers into it; the forward's saved side outputs
(norms, bitmask, pair lists) are one allocation addressed by offsets.
"""
from __future__ import annotations

import ctypes
import struct
import threading
from contextlib import contextmanager

import torch

from . import _abi

_NATIVE = {torch.float32: _abi.DTYPE_F32, torch.bfloat16: _abi.DTYPE_BF16}
_PUT = struct.Struct("<Q").pack_into  # one 64-bit device pointer into an argument template

_FWD_TENSORS = ("q1", "k1", "q2", "k2", "v", "out")
_BWD_TENSORS = ("q1", "k1", "q2", "k2", "v", "dout", "dq1", "dk1", "dq2", "dk2", "dv")
_FWD_OFF = {n: getattr(_abi.TdaFwdArgs, n).offset for n in
            _FWD_TENSORS + ("beta", "lambda_param", "norms", "occupancy", "stats", "workspace", "pairs", "zero")}
_BWD_OFF = {n: getattr(_abi.TdaBwdArgs, n).offset for n in
            _BWD_TENSORS + ("beta", "lambda_param", "dbeta", "dlambda", "norms", "occupancy", "workspace",
                            "stats", "pairs")}
_PLAN_CAP = 512  # cached argument templates (configurations) before the cache is cleared
_plans: dict = {}
_plans_lock = threading.Lock()


def _cached(key, build):
    plan = _plans.get(key)
    if plan is None:
        plan = build()
        with _plans_lock:
            if len(_plans) >= _PLAN_CAP:
                _plans.clear()
            _plans[key] = plan
    return plan


# ------------------------------------------------------------------ training-step options
_prealloc = threading.local()


def set_grad_prealloc(enabled: bool) -> None:
    """Whether a bf16 forward that will be differentiated allocates the backward's gradient
    buffers itself and clears them while its matrix-core pass runs (default True).  The
    backward then stores only the gradient rows a non-zero weight reaches, which saves about
    20 us per step at B4 H16 N4096 d128 (the zero rows' HBM writes).  The cost is memory: the
    buffers (one per input that needs a gradient: 5 x the size of q1 for the differential form,
    320 MiB at that shape) are held from the forward until the backward, on top of the saved
    inputs.  Turn it off when many layers' activations must fit at once; the backward then
    allocates the gradients itself and stores every row.  Per thread; see grad_prealloc()."""
    _prealloc.on = bool(enabled)


def grad_prealloc_enabled() -> bool:
    return getattr(_prealloc, "on", True)


@contextmanager
def grad_prealloc(enabled: bool):
    """Context manager form of set_grad_prealloc (restores the previous setting)."""
    prev = grad_prealloc_enabled()
    set_grad_prealloc(enabled)
    try:
        yield
    finally:
        set_grad_prealloc(prev)


# ------------------------------------------------------------------ tensors
def _tensor(t: torch.Tensor | None) -> _abi.TdaTensor:
    x = _abi.TdaTensor()
    if t is None:
        return x
    x.data = t.data_ptr()
    for k in range(4):
        x.stride[k] = t.stride(k)
    return x


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


_stride_ok: dict = {}


def _usable(t: torch.Tensor) -> torch.Tensor:
    """Return t itself when the kernels can read it in place (last-dim stride 1, 16-byte
    aligned base and strides), else a contiguous copy."""
    key = (t.stride(), t.element_size())
    ok = _stride_ok.get(key)
    if ok is None:
        st, es = key
        ok = _stride_ok[key] = st[3] == 1 and all(s >= 0 and (s * es) % 16 == 0 for s in st[:3])
    return t if ok and t.data_ptr() % 16 == 0 else t.contiguous()


def _empty_like_layout(t: torch.Tensor) -> torch.Tensor:
    """Uninitialised tensor of t's shape and dtype, in (B, N, H, d) memory order when t is a
    view with heads inner to the sequence (e.g. of a fused projection output), else contiguous
    (B, H, N, d).  The kernels take either through their strides."""
    b, h, n, d = t.shape
    if h > 1 and n > 1 and t.stride(1) < t.stride(2):
        return torch.empty((b, n, h, d), dtype=t.dtype, device=t.device).transpose(1, 2)
    return torch.empty(t.shape, dtype=t.dtype, device=t.device)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_inputs(tensors, names, kv_from: int | None = None):
    """Every tensor 4-D with the first one's shape, dtype and device; with kv_from, tensors
    from that index on (keys and values) may differ from it in the sequence length only."""
    ref = tensors[0]
    if not isinstance(ref, torch.Tensor):
        raise TypeError(f"{names[0]} must be a torch.Tensor")
    if ref.dim() != 4:
        raise ValueError(f"{names[0]} must have shape (batch, heads, seq_len, head_dim), got {tuple(ref.shape)}")
    shape, dtype, device = ref.shape, ref.dtype, ref.device
    kv_shape = None
    for idx, t in enumerate(tensors):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{names[idx]} must be a torch.Tensor")
        if kv_from is not None and idx >= kv_from:
            if t.dim() != 4 or t.shape[:2] != shape[:2] or t.shape[3] != shape[3]:
                raise ValueError(f"shape mismatch: {names[0]} {tuple(shape)} vs {names[idx]} {tuple(t.shape)} "
                                 "(keys and values may differ from the queries in seq_len only)")
            if kv_shape is None:
                kv_shape = t.shape
            elif t.shape != kv_shape:
                raise ValueError(f"shape mismatch: {names[kv_from]} {tuple(kv_shape)} vs {names[idx]} {tuple(t.shape)}")
        elif t.shape != shape:
            raise ValueError(f"shape mismatch: {names[0]} {tuple(shape)} vs {names[idx]} {tuple(t.shape)}")
        if t.dtype != dtype:
            raise ValueError(f"dtype mismatch: {names[0]} {dtype} vs {names[idx]} {t.dtype}")
        if t.device != device:
            raise ValueError(f"device mismatch: {names[0]} {device} vs {names[idx]} {t.device}")
    if device.type != "cuda":
        raise ValueError(f"tda_amd runs on the GPU only (HIP); got tensors on {device}")
    if not dtype.is_floating_point:
        raise ValueError(f"floating-point inputs required, got {dtype}")


def _common(args, t: torch.Tensor, branches: int, normalize: bool, relu_power: float,
            n_kv: int | None = None, q_offset: int = 0):
    b, h, n, d = t.shape
    args.seq_len_kv = n if n_kv is None else n_kv
    args.q_offset = q_offset
    args.abi_version = _abi.ABI_VERSION
    args.dtype = _NATIVE[t.dtype]
    args.branches = branches
    args.normalize = 1 if normalize else 0
    args.causal = 1
    args.relu_power = float(relu_power)
    args.batch, args.heads, args.seq_len, args.head_dim = b, h, n, d


# ------------------------------------------------------------------ argument templates
def _fwd_template(ts, branches, normalize, relu_power, q_offset, zero_bytes):
    """(template bytes, workspace bytes) of tda_fwd for tensors ts = (q1, k1, q2, k2, v, out)
    (q2, k2 None for one branch): every field but the device pointers."""
    q1, k1 = ts[0], ts[1]
    key = ("fwd", q1.shape, k1.shape[2], q1.dtype, branches, bool(normalize), float(relu_power), q_offset,
           zero_bytes, tuple(None if t is None else t.stride() for t in ts))

    def build():
        a = _abi.TdaFwdArgs()
        _common(a, q1, branches, normalize, relu_power, k1.shape[2], q_offset)
        for name, t in zip(_FWD_TENSORS, ts):
            if t is not None:
                getattr(a, name).stride[:] = t.stride()
        a.zero_bytes = zero_bytes
        ws = _abi.load().tda_fwd_workspace_bytes_for(ctypes.byref(a))
        a.workspace_bytes = (ws + 255) // 256 * 256
        return bytes(a), a.workspace_bytes

    return _cached(key, build)


def _bwd_template(ts, branches, normalize, relu_power, q_offset, zeroed):
    """(template bytes, workspace bytes) of tda_bwd for ts in _BWD_TENSORS order."""
    q1, k1 = ts[0], ts[1]
    key = ("bwd", q1.shape, k1.shape[2], q1.dtype, branches, bool(normalize), float(relu_power), q_offset,
           bool(zeroed), tuple(None if t is None else t.stride() for t in ts))

    def build():
        a = _abi.TdaBwdArgs()
        _common(a, q1, branches, normalize, relu_power, k1.shape[2], q_offset)
        for name, t in zip(_BWD_TENSORS, ts):
            if t is not None:
                getattr(a, name).stride[:] = t.stride()
        a.grads_zeroed = 1 if zeroed else 0
        b, h, n, d = q1.shape
        a.workspace_bytes = (_abi.load().tda_bwd_workspace_bytes(b, h, n, d) + 255) // 256 * 256
        return bytes(a), a.workspace_bytes

    return _cached(key, build)


def _fill(buf: bytearray, off: dict, names, tensors) -> None:
    for name, t in zip(names, tensors):
        if t is not None:
            _PUT(buf, off[name], t.data_ptr())


def _launch(fn, args_type, buf: bytearray, device, what: str) -> None:
    a = args_type.from_buffer(buf)
    with torch.cuda.device(device):
        _abi.check(fn(ctypes.byref(a), _stream(device)), what)


# ------------------------------------------------------------------ forward / backward calls
def _forward_raw(q1, k1, q2, k2, v, out, beta, lam, relu_power, normalize, branches, q_offset,
                 norms_p=0, occ_p=0, stats_p=0, pairs_p=0, zero_p=0, zero_bytes=0, no_alloc=False):
    """One tda_fwd (tda_fwd_noalloc) call on usable tensors with the side outputs given as
    device addresses (0: none)."""
    lib = _abi.load()
    ts = (q1, k1, q2, k2, v, out) if branches == 2 else (q1, k1, None, None, v, out)
    tpl, ws_bytes = _fwd_template(ts, branches, normalize, relu_power, q_offset, zero_bytes)
    buf = bytearray(tpl)
    _fill(buf, _FWD_OFF, _FWD_TENSORS, ts)
    _PUT(buf, _FWD_OFF["beta"], beta.data_ptr())
    if branches == 2:
        _PUT(buf, _FWD_OFF["lambda_param"], lam.data_ptr())
    for name, p in (("norms", norms_p), ("occupancy", occ_p), ("stats", stats_p), ("pairs", pairs_p),
                    ("zero", zero_p)):
        if p:
            _PUT(buf, _FWD_OFF[name], p)
    if no_alloc:
        _PUT(buf, _FWD_OFF["workspace"], 0)
        struct.pack_into("<Q", buf, _abi.TdaFwdArgs.workspace_bytes.offset, 0)
        _launch(lib.tda_fwd_noalloc, _abi.TdaFwdArgs, buf, q1.device, "tda_fwd_noalloc")
        return
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q1.device)
    _PUT(buf, _FWD_OFF["workspace"], ws.data_ptr())
    _launch(lib.tda_fwd, _abi.TdaFwdArgs, buf, q1.device, "tda_fwd")


def forward(q1, k1, q2, k2, v, beta, lam, relu_power: float, normalize: bool, branches: int,
            norms=None, occupancy=None, stats=None, q_offset: int = 0, pairs=None,
            out=None, no_alloc: bool = False, zero=None) -> torch.Tensor:
    """One forward launch.  Tensors must already be in a native dtype (float32 / bfloat16)
    on one device; beta (and lam) are 0-dim float32 tensors on that device.  q1 (q2) have Nq
    rows at positions q_offset.., k1 (k2) and v have Nk rows.  The optional norms /
    occupancy / stats / pairs buffers receive the side outputs described in include/tda.h.
    no_alloc: call tda_fwd_noalloc, whose workspace is the library's own device array (no
    workspace tensor here); with `out` (and `norms` when normalize) given, the call then
    allocates nothing.  zero: a contiguous tensor the call sets to zero (the gradient buffer
    of grad_buffers, cleared while the forward runs)."""
    lib = _abi.load()
    q1, k1, v = _usable(q1), _usable(k1), _usable(v)
    if branches == 2:
        q2, k2 = _usable(q2), _usable(k2)
    if out is None:
        out = _empty_like_layout(q1)
    elif out.shape != q1.shape or out.dtype != q1.dtype or out.device != q1.device:
        raise ValueError("out must match q1's shape, dtype and device")
    nk = k1.shape[2]
    if normalize and norms is None:  # scratch: the kernels need the row norms either way
        norms = torch.empty(lib.tda_norms_floats_kv(*q1.shape[:3], nk, branches), dtype=torch.float32,
                            device=q1.device)
    if stats is not None and (stats.dtype != torch.int64 or stats.numel() < 3 or stats.device != q1.device):
        raise ValueError("stats must be an int64 tensor of at least 3 elements on the inputs' device")
    zero_p = zero_bytes = 0
    if zero is not None:
        if not zero.is_contiguous() or zero.device != q1.device:
            raise ValueError("zero must be a contiguous tensor on the inputs' device")
        zero_p, zero_bytes = zero.data_ptr(), zero.numel() * zero.element_size()
    _forward_raw(q1, k1, q2, k2, v, out, beta, lam, relu_power, normalize, branches, q_offset,
                 _ptr(norms) or 0, _ptr(occupancy) or 0, _ptr(stats) or 0, _ptr(pairs) or 0, zero_p, zero_bytes,
                 no_alloc)
    return out


def _grad_views(buf: torch.Tensor, srcs):
    """Views of one flat buffer with the shapes (and the memory order _empty_like_layout would
    give) of the tensors in srcs (None entries stay None)."""
    views, off = [], 0
    for t in srcs:
        if t is None:
            views.append(None)
            continue
        b, h, s, d = t.shape
        n = t.numel()
        flat = buf[off:off + n]
        off += n
        if h > 1 and s > 1 and t.stride(1) < t.stride(2):
            views.append(flat.view(b, s, h, d).transpose(1, 2))
        else:
            views.append(flat.view(b, h, s, d))
    return views


def grad_buffers(q1, k1, q2, k2, v, branches: int):
    """One allocation holding the backward's gradient tensors: returns (buffer, [dq1, dk1,
    dq2, dk2, dv]) with the branch-2 entries None when branches == 1.  Each gradient has its
    input's shape and dtype, in the memory order _empty_like_layout would give it; the forward
    can clear the whole buffer (its `zero` argument) and the backward then stores only the
    non-zero rows (grads=)."""
    srcs = [q1, k1, q2, k2, v] if branches == 2 else [q1, k1, None, None, v]
    buf = torch.empty(sum(0 if t is None else t.numel() for t in srcs), dtype=q1.dtype, device=q1.device)
    return buf, _grad_views(buf, srcs)


def _backward_raw(q1, k1, q2, k2, v, dout, grads, beta, lam, relu_power, normalize, branches, q_offset,
                  norms_p, occ_p, pairs_p, stats_p, zeroed):
    """One tda_bwd call on usable tensors into grads = [dq1, dk1, dq2, dk2, dv]; returns
    (dbeta, dlambda) (dlambda None for one branch)."""
    lib = _abi.load()
    dq1, dk1, dq2, dk2, dv = grads
    if branches == 2:
        ts = (q1, k1, q2, k2, v, dout, dq1, dk1, dq2, dk2, dv)
    else:
        ts = (q1, k1, None, None, v, dout, dq1, dk1, None, None, dv)
    tpl, ws_bytes = _bwd_template(ts, branches, normalize, relu_power, q_offset, zeroed)
    buf = bytearray(tpl)
    _fill(buf, _BWD_OFF, _BWD_TENSORS, ts)
    # dbeta, dlambda and the workspace in one allocation: the scalars at floats 0 and 1, the
    # workspace from byte 256
    scal = torch.empty(64 + ws_bytes // 4, dtype=torch.float32, device=q1.device)
    base = scal.data_ptr()
    dbeta = scal[0]
    dlam = scal[1] if branches == 2 else None
    _PUT(buf, _BWD_OFF["dbeta"], base)
    _PUT(buf, _BWD_OFF["beta"], beta.data_ptr())
    if branches == 2:
        _PUT(buf, _BWD_OFF["dlambda"], base + 4)
        _PUT(buf, _BWD_OFF["lambda_param"], lam.data_ptr())
    _PUT(buf, _BWD_OFF["workspace"], base + 256)
    for name, p in (("norms", norms_p), ("occupancy", occ_p), ("pairs", pairs_p), ("stats", stats_p)):
        if p:
            _PUT(buf, _BWD_OFF[name], p)
    _launch(lib.tda_bwd, _abi.TdaBwdArgs, buf, q1.device, "tda_bwd")
    return dbeta, dlam


def backward(q1, k1, q2, k2, v, dout, beta, lam, relu_power: float, normalize: bool,
             branches: int, norms=None, occupancy=None, stats=None, q_offset: int = 0, pairs=None,
             grads=None):
    """One backward launch: returns (dq1, dk1, dq2, dk2, dv, dbeta, dlambda); the branch-2
    entries and dlambda are None when branches == 1.  pairs: the forward's pair lists (bf16,
    with occupancy), or None for the bitmask tiles alone.  grads: the [dq1, dk1, dq2, dk2, dv]
    of grad_buffers whose buffer the forward cleared; the call then stores only the gradient
    rows some non-zero weight reaches."""
    q1, k1, v, dout = _usable(q1), _usable(k1), _usable(v), _usable(dout)
    if branches == 2:
        q2, k2 = _usable(q2), _usable(k2)
    if grads is not None:
        gl = list(grads)
    else:
        gl = [_empty_like_layout(q1), _empty_like_layout(k1), None, None, _empty_like_layout(v)]
        if branches == 2:
            gl[2], gl[3] = _empty_like_layout(q2), _empty_like_layout(k2)
    dbeta, dlam = _backward_raw(q1, k1, q2, k2, v, dout, gl, beta, lam, relu_power, normalize, branches, q_offset,
                                _ptr(norms) or 0, _ptr(occupancy) or 0, _ptr(pairs) or 0, _ptr(stats) or 0,
                                grads is not None)
    return gl[0], gl[1], gl[2], gl[3], gl[4], dbeta, dlam


def side_buffers(shape, branches: int, normalize: bool, device, n_kv: int | None = None):
    """Allocate the forward's norms and occupancy outputs (uninitialised: the forward writes
    every element); shape is the queries' (B, H, Nq, d), n_kv the key rows (default Nq)."""
    lib = _abi.load()
    b, h, n, _ = shape
    nk = n if n_kv is None else n_kv
    occ = torch.empty(lib.tda_occupancy_words_kv(b, h, n, nk, branches), dtype=torch.int32, device=device)
    norms = (torch.empty(lib.tda_norms_floats_kv(b, h, n, nk, branches), dtype=torch.float32, device=device)
             if normalize else None)
    return norms, occ


def pair_buffer(shape, branches: int, device):
    """Allocate the forward's pair-list output (bf16 forwards write it; uninitialised: the
    forward writes every count it sets a list by)."""
    b, h, n, _ = shape
    return torch.empty(_abi.load().tda_pair_words(b, h, n, branches), dtype=torch.int32, device=device)


def _saved_layout(shape, nk: int, branches: int, normalize: bool, pairs: bool):
    """Byte offsets (norms, occupancy, pairs; -1: absent) and total bytes of the forward's saved
    side outputs in one allocation (each part 256-byte aligned)."""
    key = ("saved", tuple(shape), nk, branches, normalize, pairs)

    def build():
        lib = _abi.load()
        b, h, n, _ = shape
        parts = [lib.tda_norms_floats_kv(b, h, n, nk, branches) * 4 if normalize else 0,
                 lib.tda_occupancy_words_kv(b, h, n, nk, branches) * 4,
                 lib.tda_pair_words(b, h, n, branches) * 4 if pairs else 0]
        offs, total = [], 0
        for nbytes in parts:
            if nbytes:
                offs.append(total)
                total += (nbytes + 255) // 256 * 256
            else:
                offs.append(-1)
        return tuple(offs), total

    return _cached(key, build)


class TDAFunction(torch.autograd.Function):
    """Autograd node for TRA (branches == 1) and fused TDA (branches == 2).

    forward(ctx, q1, k1, q2, k2, v, beta, lam, relu_power, normalize, branches):
    q2, k2, lam are None when branches == 1; beta / lam are 0-dim float32 device tensors.
    The saved side outputs (norms, bitmask, bf16 pair lists) share one allocation; with
    grad_prealloc on (bf16, every input needing a gradient) the forward also allocates the
    gradients and clears them (see set_grad_prealloc)."""

    @staticmethod
    def forward(ctx, q1, k1, q2, k2, v, beta, lam, relu_power, normalize, branches, q_offset=0):
        ng = ctx.needs_input_grad
        need = ng[0] or ng[1] or ng[2] or ng[3] or ng[4] or ng[5] or ng[6]
        q1, k1, v = _usable(q1), _usable(k1), _usable(v)
        if branches == 2:
            q2, k2 = _usable(q2), _usable(k2)
        dev = q1.device
        out = _empty_like_layout(q1)
        nk = k1.shape[2]
        bf16 = q1.dtype == torch.bfloat16
        saved = gbuf = None
        norms_p = occ_p = pairs_p = zero_p = zero_bytes = 0
        # pair lists: written by the bf16 forward and by the fp32 candidate pass (normalised, more
        # than one query tile); head_dim 256 has its own kernels, which use none
        want_pairs = need and q1.shape[3] <= 128 and (bf16 or (normalize and q1.shape[2] > 32))
        if need or normalize:
            (o_n, o_o, o_p), total = _saved_layout(q1.shape, nk, branches, normalize, want_pairs)
            saved = torch.empty(total, dtype=torch.uint8, device=dev)
            base = saved.data_ptr()
            norms_p = base + o_n if o_n >= 0 else 0
            if need:
                occ_p = base + o_o
                pairs_p = base + o_p if o_p >= 0 else 0
        all_inputs = ng[0] and ng[1] and ng[4] and (branches == 1 or (ng[2] and ng[3]))
        if need and bf16 and all_inputs and grad_prealloc_enabled():
            # the gradients, cleared by this forward while its matrix-core pass runs: the pair
            # backward then stores only the rows a non-zero weight reaches
            srcs = [q1, k1, q2, k2, v] if branches == 2 else [q1, k1, None, None, v]
            gbuf = torch.empty(sum(0 if t is None else t.numel() for t in srcs), dtype=q1.dtype, device=dev)
            zero_p, zero_bytes = gbuf.data_ptr(), gbuf.numel() * gbuf.element_size()
        _forward_raw(q1, k1, q2, k2, v, out, beta, lam, relu_power, normalize, branches, q_offset,
                     norms_p, occ_p, 0, pairs_p, zero_p, zero_bytes)
        if need:
            ctx.save_for_backward(q1, k1, q2, k2, v, beta, lam)
            ctx.saved = saved  # side outputs: not inputs or outputs of the node
            ctx.gbuf = gbuf
            ctx.ptrs = (norms_p, occ_p, pairs_p)
            ctx.cfg = (float(relu_power), bool(normalize), int(branches), int(q_offset))
        return out

    @staticmethod
    def backward(ctx, dout):
        q1, k1, q2, k2, v, beta, lam = ctx.saved_tensors
        relu_power, normalize, branches, q_offset = ctx.cfg
        norms_p, occ_p, pairs_p = ctx.ptrs
        if dout.dtype != q1.dtype:
            dout = dout.to(q1.dtype)
        dout = _usable(dout)
        # the cleared gradient buffers serve the first backward only (a second one, under
        # retain_graph, must not overwrite gradients already handed out)
        gbuf, ctx.gbuf = ctx.gbuf, None
        if gbuf is not None:
            grads = _grad_views(gbuf, [q1, k1, q2, k2, v] if branches == 2 else [q1, k1, None, None, v])
        else:
            grads = [_empty_like_layout(q1), _empty_like_layout(k1), None, None, _empty_like_layout(v)]
            if branches == 2:
                grads[2], grads[3] = _empty_like_layout(q2), _empty_like_layout(k2)
        dbeta, dlam = _backward_raw(q1, k1, q2, k2, v, dout, grads, beta, lam, relu_power, normalize, branches,
                                    q_offset, norms_p, occ_p, pairs_p, 0, gbuf is not None)
        ng = ctx.needs_input_grad
        dq1, dk1, dq2, dk2, dv = grads
        return (dq1 if ng[0] else None, dk1 if ng[1] else None,
                dq2 if ng[2] else None, dk2 if ng[3] else None,
                dv if ng[4] else None, dbeta if ng[5] else None,
                dlam if (branches == 2 and ng[6]) else None, None, None, None, None)
