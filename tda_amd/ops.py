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
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi

_NATIVE = {torch.float32: _abi.DTYPE_F32, torch.bfloat16: _abi.DTYPE_BF16}


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


def _usable(t: torch.Tensor) -> torch.Tensor:
    """Return t itself when the kernels can read it in place (last-dim stride 1, 16-byte
    aligned base and strides), else a contiguous copy."""
    es = t.element_size()
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0
          and all(s >= 0 and (s * es) % 16 == 0 for s in t.stride()[:3]))
    return t if ok else t.contiguous()


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
    kv_ref = tensors[kv_from] if kv_from is not None else None
    for idx, (t, n) in enumerate(zip(tensors, names)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{n} must be a torch.Tensor")
        want = ref.shape
        if kv_from is not None and idx >= kv_from:
            if t.dim() != 4 or t.shape[:2] != ref.shape[:2] or t.shape[3] != ref.shape[3]:
                raise ValueError(f"shape mismatch: {names[0]} {tuple(ref.shape)} vs {n} {tuple(t.shape)} "
                                 "(keys and values may differ from the queries in seq_len only)")
            want = kv_ref.shape
        if t.shape != want:
            raise ValueError(f"shape mismatch: {names[kv_from if kv_from is not None and idx >= kv_from else 0]} "
                             f"{tuple(want)} vs {n} {tuple(t.shape)}")
        if t.dtype != ref.dtype:
            raise ValueError(f"dtype mismatch: {names[0]} {ref.dtype} vs {n} {t.dtype}")
        if t.device != ref.device:
            raise ValueError(f"device mismatch: {names[0]} {ref.device} vs {n} {t.device}")
    if ref.device.type != "cuda":
        raise ValueError(f"tda_amd runs on the GPU only (HIP); got tensors on {ref.device}")
    if not ref.dtype.is_floating_point:
        raise ValueError(f"floating-point inputs required, got {ref.dtype}")


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
    a = _abi.TdaFwdArgs()
    nk = k1.shape[2]
    _common(a, q1, branches, normalize, relu_power, nk, q_offset)
    a.q1, a.k1, a.v, a.out = _tensor(q1), _tensor(k1), _tensor(v), _tensor(out)
    if branches == 2:
        a.q2, a.k2 = _tensor(q2), _tensor(k2)
    a.beta = _ptr(beta)
    a.lambda_param = _ptr(lam) if branches == 2 else None
    if normalize and norms is None:  # scratch: the kernels need the row norms either way
        norms = torch.empty(lib.tda_norms_floats_kv(*q1.shape[:3], nk, branches), dtype=torch.float32,
                            device=q1.device)
    if stats is not None and (stats.dtype != torch.int64 or stats.numel() < 3 or stats.device != q1.device):
        raise ValueError("stats must be an int64 tensor of at least 3 elements on the inputs' device")
    a.norms, a.occupancy, a.stats, a.pairs = _ptr(norms), _ptr(occupancy), _ptr(stats), _ptr(pairs)
    if zero is not None:
        if not zero.is_contiguous() or zero.device != q1.device:
            raise ValueError("zero must be a contiguous tensor on the inputs' device")
        a.zero, a.zero_bytes = zero.data_ptr(), zero.numel() * zero.element_size()
    if no_alloc:
        with torch.cuda.device(q1.device):
            _abi.check(lib.tda_fwd_noalloc(ctypes.byref(a), _stream(q1.device)), "tda_fwd_noalloc")
        return out
    ws = torch.empty((lib.tda_fwd_workspace_bytes_for(ctypes.byref(a)) + 3) // 4,
                     dtype=torch.float32, device=q1.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    with torch.cuda.device(q1.device):
        _abi.check(lib.tda_fwd(ctypes.byref(a), _stream(q1.device)), "tda_fwd")
    return out


def grad_buffers(q1, k1, q2, k2, v, branches: int):
    """One allocation holding the backward's gradient tensors: returns (buffer, [dq1, dk1,
    dq2, dk2, dv]) with the branch-2 entries None when branches == 1.  Each gradient has its
    input's shape and dtype, in the memory order _empty_like_layout would give it; the forward
    can clear the whole buffer (its `zero` argument) and the backward then stores only the
    non-zero rows (grads=)."""
    srcs = [q1, k1, q2, k2, v] if branches == 2 else [q1, k1, None, None, v]
    sizes = [0 if t is None else t.numel() for t in srcs]
    buf = torch.empty(sum(sizes), dtype=q1.dtype, device=q1.device)
    views, off = [], 0
    for t, n in zip(srcs, sizes):
        if t is None:
            views.append(None)
            continue
        flat = buf[off:off + n]
        off += n
        b, h, s, d = t.shape
        if h > 1 and s > 1 and t.stride(1) < t.stride(2):
            views.append(flat.view(b, s, h, d).transpose(1, 2))
        else:
            views.append(flat.view(b, h, s, d))
    return buf, views


def backward(q1, k1, q2, k2, v, dout, beta, lam, relu_power: float, normalize: bool,
             branches: int, norms=None, occupancy=None, stats=None, q_offset: int = 0, pairs=None,
             grads=None):
    """One backward launch: returns (dq1, dk1, dq2, dk2, dv, dbeta, dlambda); the branch-2
    entries and dlambda are None when branches == 1.  pairs: the forward's pair lists (bf16,
    with occupancy), or None for the bitmask tiles alone.  grads: the [dq1, dk1, dq2, dk2, dv]
    of grad_buffers whose buffer the forward cleared; the call then stores only the gradient
    rows some non-zero weight reaches."""
    lib = _abi.load()
    q1, k1, v, dout = _usable(q1), _usable(k1), _usable(v), _usable(dout)
    if branches == 2:
        q2, k2 = _usable(q2), _usable(k2)
    dev = q1.device
    dq2 = dk2 = dlam = None
    if grads is not None:
        dq1, dk1, dq2, dk2, dv = grads
    else:
        dq1, dk1, dv = _empty_like_layout(q1), _empty_like_layout(k1), _empty_like_layout(v)
        if branches == 2:
            dq2, dk2 = _empty_like_layout(q2), _empty_like_layout(k2)
    if branches == 2:
        dlam = torch.empty((), dtype=torch.float32, device=dev)
    dbeta = torch.empty((), dtype=torch.float32, device=dev)
    b, h, n, d = q1.shape
    ws_bytes = lib.tda_bwd_workspace_bytes(b, h, n, d)
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev)
    a = _abi.TdaBwdArgs()
    _common(a, q1, branches, normalize, relu_power, k1.shape[2], q_offset)
    a.q1, a.k1, a.v, a.dout = _tensor(q1), _tensor(k1), _tensor(v), _tensor(dout)
    a.dq1, a.dk1, a.dv = _tensor(dq1), _tensor(dk1), _tensor(dv)
    if branches == 2:
        a.q2, a.k2, a.dq2, a.dk2 = _tensor(q2), _tensor(k2), _tensor(dq2), _tensor(dk2)
    a.beta = _ptr(beta)
    a.lambda_param = _ptr(lam) if branches == 2 else None
    a.dbeta, a.dlambda = _ptr(dbeta), _ptr(dlam)
    a.norms, a.occupancy, a.pairs = _ptr(norms), _ptr(occupancy), _ptr(pairs)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    a.stats = _ptr(stats)
    a.grads_zeroed = 1 if grads is not None else 0
    with torch.cuda.device(dev):
        _abi.check(lib.tda_bwd(ctypes.byref(a), _stream(dev)), "tda_bwd")
    return dq1, dk1, dq2, dk2, dv, dbeta, dlam


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


class TDAFunction(torch.autograd.Function):
    """Autograd node for TRA (branches == 1) and fused TDA (branches == 2).

    forward(ctx, q1, k1, q2, k2, v, beta, lam, relu_power, normalize, branches):
    q2, k2, lam are None when branches == 1; beta / lam are 0-dim float32 device tensors."""

    @staticmethod
    def forward(ctx, q1, k1, q2, k2, v, beta, lam, relu_power, normalize, branches, q_offset=0):
        need = any(ctx.needs_input_grad[:7])
        norms = occ = pairs = gbuf = None
        grads = [None] * 5
        if need:
            norms, occ = side_buffers(q1.shape, branches, normalize, q1.device, k1.shape[2])
            if q1.dtype == torch.bfloat16:
                pairs = pair_buffer(q1.shape, branches, q1.device)
                # the gradients, cleared by this forward while its matrix-core pass runs: the
                # pair backward then stores only the rows a non-zero weight reaches
                gbuf, grads = grad_buffers(q1, k1, q2, k2, v, branches)
        out = forward(q1, k1, q2, k2, v, beta, lam, relu_power, normalize, branches, norms, occ,
                      q_offset=q_offset, pairs=pairs, zero=gbuf)
        ctx.save_for_backward(q1, k1, q2, k2, v, beta, lam, norms, occ, pairs, *grads)
        ctx.cfg = (float(relu_power), bool(normalize), int(branches), int(q_offset), gbuf is not None)
        return out

    @staticmethod
    def backward(ctx, dout):
        q1, k1, q2, k2, v, beta, lam, norms, occ, pairs, *grads = ctx.saved_tensors
        relu_power, normalize, branches, q_offset, zeroed = ctx.cfg
        dout = dout.to(q1.dtype)
        dq1, dk1, dq2, dk2, dv, dbeta, dlam = backward(
            q1, k1, q2, k2, v, dout, beta, lam, relu_power, normalize, branches, norms, occ,
            q_offset=q_offset, pairs=pairs, grads=grads if zeroed else None)
        ng = ctx.needs_input_grad
        return (dq1 if ng[0] else None, dk1 if ng[1] else None,
                dq2 if ng[2] else None, dk2 if ng[3] else None,
                dv if ng[4] else None, dbeta if ng[5] else None,
                dlam if (branches == 2 and ng[6]) else None, None, None, None, None)
