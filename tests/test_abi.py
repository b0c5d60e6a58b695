"""C-ABI tests that need no GPU: the library loads, exports every function include/tda.h
declares, the ctypes mirror matches the C struct layout, and every invalid argument maps to
its error code without touching a device."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest
import torch

from tda_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tda.h")


def _lib():
    if not os.path.exists(_abi.lib_path()):
        pytest.skip("libtda_hip.so not built (python -m tda_amd.build)")
    return _abi.load()


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tda_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_api():
    names = _declared_functions()
    assert set(names) == set(_abi.SIGNATURES), names


def test_library_exports_every_declared_symbol():
    lib = _lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.tda_abi_version() == _abi.ABI_VERSION


def test_struct_layout_matches_c_header(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc missing")
    fields = {
        "tda_fwd_args": _abi.TdaFwdArgs, "tda_bwd_args": _abi.TdaBwdArgs, "tda_tensor": _abi.TdaTensor,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, py in fields.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln:
            c, f, v = ln.split()
            got[(c, f)] = int(v)
    for cname, py in fields.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, (cname, f)


FAKE = 0x10000  # aligned, never dereferenced: validation is host-only


def _tensor(shape, es=2, strides=None):
    t = _abi.TdaTensor()
    t.data = FAKE
    b, h, n, d = shape
    st = strides or (h * n * d, n * d, d, 1)
    for k in range(4):
        t.stride[k] = st[k]
    return t


def _fwd_args(shape=(2, 3, 100, 128), branches=2, dtype=_abi.DTYPE_BF16):
    a = _abi.TdaFwdArgs()
    a.abi_version, a.dtype, a.branches, a.normalize, a.causal = _abi.ABI_VERSION, dtype, branches, 1, 1
    a.relu_power = 2.0
    a.batch, a.heads, a.seq_len, a.head_dim = shape
    for f in ("q1", "k1", "q2", "k2", "v", "out"):
        setattr(a, f, _tensor(shape))
    a.beta = FAKE
    a.lambda_param = FAKE
    a.norms = FAKE
    a.workspace = FAKE
    a.workspace_bytes = _lib().tda_fwd_workspace_bytes(*shape[:3], branches)
    return a


def _bwd_args(shape=(2, 3, 100, 128), branches=2):
    lib = _lib()
    a = _abi.TdaBwdArgs()
    a.abi_version, a.dtype, a.branches, a.normalize, a.causal = _abi.ABI_VERSION, _abi.DTYPE_BF16, branches, 1, 1
    a.relu_power = 2.0
    a.batch, a.heads, a.seq_len, a.head_dim = shape
    for f in ("q1", "k1", "q2", "k2", "v", "dout", "dq1", "dk1", "dq2", "dk2", "dv"):
        setattr(a, f, _tensor(shape))
    a.beta = a.lambda_param = a.norms = FAKE
    a.workspace = FAKE
    a.workspace_bytes = lib.tda_bwd_workspace_bytes(*shape)
    return a


def test_valid_args_pass():
    lib = _lib()
    assert lib.tda_validate_fwd(ctypes.byref(_fwd_args())) == _abi.OK
    assert lib.tda_validate_fwd(ctypes.byref(_fwd_args(branches=1, dtype=_abi.DTYPE_F32))) == _abi.OK
    assert lib.tda_validate_bwd(ctypes.byref(_bwd_args())) == _abi.OK


@pytest.mark.parametrize("mutate,code", [
    (lambda a: setattr(a, "abi_version", 99), _abi.ERR_ABI),
    (lambda a: setattr(a, "dtype", 7), _abi.ERR_DTYPE),
    (lambda a: setattr(a, "branches", 3), _abi.ERR_BRANCHES),
    (lambda a: setattr(a, "causal", 0), _abi.ERR_CAUSAL),
    (lambda a: setattr(a, "head_dim", 96), _abi.ERR_HEAD_DIM),
    (lambda a: setattr(a, "head_dim", 512), _abi.ERR_HEAD_DIM),
    (lambda a: setattr(a, "head_dim", 32), _abi.ERR_HEAD_DIM),
    (lambda a: setattr(a, "seq_len", 0), _abi.ERR_SHAPE),
    (lambda a: setattr(a, "batch", 0), _abi.ERR_SHAPE),
    (lambda a: setattr(a, "relu_power", -1.0), _abi.ERR_POWER),
    (lambda a: setattr(a, "relu_power", float("nan")), _abi.ERR_POWER),
    (lambda a: setattr(a, "relu_power", float("inf")), _abi.ERR_POWER),
    (lambda a: setattr(a, "beta", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a, "lambda_param", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a.q2, "data", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a.out, "data", None), _abi.ERR_NULL_POINTER),
    (lambda a: a.v.stride.__setitem__(3, 2), _abi.ERR_LAYOUT),
    (lambda a: a.k1.stride.__setitem__(2, 129), _abi.ERR_LAYOUT),
    (lambda a: a.q1.stride.__setitem__(0, -128), _abi.ERR_LAYOUT),
    (lambda a: setattr(a.q1, "data", FAKE + 2), _abi.ERR_LAYOUT),
    (lambda a: setattr(a, "norms", None), _abi.ERR_NORMS),
    (lambda a: a.k1.stride.__setitem__(2, (1 << 25) + 8), _abi.ERR_LAYOUT),
    (lambda a: setattr(a, "workspace", None), _abi.ERR_WORKSPACE),
    (lambda a: setattr(a, "workspace_bytes", a.workspace_bytes - 4), _abi.ERR_WORKSPACE),
    (lambda a: setattr(a, "workspace", FAKE + 8), _abi.ERR_WORKSPACE),
    (lambda a: setattr(a, "q_offset", -1), _abi.ERR_OFFSET),
    (lambda a: setattr(a, "q_offset", (1 << 30) - 64), _abi.ERR_OFFSET),  # position past 2^30 - 64
    (lambda a: setattr(a, "seq_len_kv", 1 << 30), _abi.ERR_OFFSET),
    (lambda a: setattr(a, "seq_len_kv", -5), _abi.ERR_OFFSET),
    # more key rows need a wider bitmask than the workspace holds
    (lambda a: setattr(a, "seq_len_kv", 5000), _abi.ERR_WORKSPACE),
    # the zero range: 16-byte aligned, a multiple of 16 bytes, present when its size is not 0
    (lambda a: (setattr(a, "zero", FAKE), setattr(a, "zero_bytes", 40)), _abi.ERR_LAYOUT),
    (lambda a: (setattr(a, "zero", FAKE + 8), setattr(a, "zero_bytes", 64)), _abi.ERR_LAYOUT),
    (lambda a: (setattr(a, "zero", None), setattr(a, "zero_bytes", 64)), _abi.ERR_NULL_POINTER),
])
def test_fwd_validator_rejects(mutate, code):
    lib = _lib()
    a = _fwd_args()
    mutate(a)
    assert lib.tda_validate_fwd(ctypes.byref(a)) == code
    assert lib.tda_fwd(ctypes.byref(a), None) == code  # rejected before any launch


def test_workspace_for_one_call():
    """tda_fwd_workspace_bytes_for: the int8 keys only with normalize (bf16 or fp32) and more
    than one query tile, at the call's head_dim; never above the shape-only bound."""
    lib = _lib()
    r256 = lambda b: 256 * ((b + 255) // 256)  # noqa: E731
    a = _fwd_args()  # bf16, normalize, (2, 3, 100, 128), two branches
    full = lib.tda_fwd_workspace_bytes_for(ctypes.byref(a))
    assert full == lib.tda_fwd_workspace_bytes(2, 3, 100, 2)
    a.normalize = 0
    assert full - lib.tda_fwd_workspace_bytes_for(ctypes.byref(a)) == r256(2 * 6 * 100 * 128) + r256(2 * 6 * 100 * 8)
    a.normalize, a.dtype = 1, _abi.DTYPE_F32  # the int8 screen also runs on fp32 rows
    assert lib.tda_fwd_workspace_bytes_for(ctypes.byref(a)) == lib.tda_fwd_workspace_bytes_for(
        ctypes.byref(_fwd_args(dtype=_abi.DTYPE_F32))) == full
    b = _fwd_args(shape=(2, 3, 100, 64))
    assert full - lib.tda_fwd_workspace_bytes_for(ctypes.byref(b)) == r256(2 * 6 * 100 * 128) - r256(2 * 6 * 100 * 64)
    b.seq_len, b.seq_len_kv, b.q_offset = 20, 300, 280  # one query tile: decode partials, no int8 keys
    assert lib.tda_fwd_workspace_bytes_for(ctypes.byref(b)) == lib.tda_fwd_workspace_bytes_kv(2, 3, 20, 300, 2)
    b.head_dim = 96
    assert lib.tda_fwd_workspace_bytes_for(ctypes.byref(b)) == 0
    assert lib.tda_fwd_workspace_bytes_for(None) == 0
    w = _fwd_args(shape=(2, 3, 100, 256))  # head_dim 256 has no screen: no int8 keys
    a.normalize, a.dtype = 0, _abi.DTYPE_BF16
    assert lib.tda_fwd_workspace_bytes_for(ctypes.byref(w)) == lib.tda_fwd_workspace_bytes_for(ctypes.byref(a))
    assert lib.tda_validate_fwd(ctypes.byref(w)) == _abi.OK


def test_zero_range_args_pass():
    lib = _lib()
    a = _fwd_args()
    a.zero, a.zero_bytes = FAKE, 1 << 20
    assert lib.tda_validate_fwd(ctypes.byref(a)) == _abi.OK
    a.zero, a.zero_bytes = None, 0
    assert lib.tda_validate_fwd(ctypes.byref(a)) == _abi.OK
    b = _bwd_args()
    b.grads_zeroed = 1
    assert lib.tda_validate_bwd(ctypes.byref(b)) == _abi.OK


def test_offset_args_pass():
    """seq_len_kv = 0 means Nk = Nq; a KV-cache shape with its workspace validates."""
    lib = _lib()
    a = _fwd_args()
    a.seq_len_kv, a.q_offset = 0, 0
    assert lib.tda_validate_fwd(ctypes.byref(a)) == _abi.OK
    a.seq_len, a.seq_len_kv, a.q_offset = 1, 900, 899
    a.workspace_bytes = lib.tda_fwd_workspace_bytes_kv(2, 3, 1, 900, 2)
    assert lib.tda_validate_fwd(ctypes.byref(a)) == _abi.OK
    b = _bwd_args()
    b.seq_len, b.seq_len_kv, b.q_offset = 7, 300, 100
    b.workspace_bytes = lib.tda_bwd_workspace_bytes(2, 3, 7, 128)
    assert lib.tda_validate_bwd(ctypes.byref(b)) == _abi.OK
    b.q_offset = -3
    assert lib.tda_validate_bwd(ctypes.byref(b)) == _abi.ERR_OFFSET


def test_single_branch_ignores_second_branch_pointers():
    lib = _lib()
    a = _fwd_args(branches=1)
    a.q2.data = None
    a.lambda_param = None
    assert lib.tda_validate_fwd(ctypes.byref(a)) == _abi.OK


def test_zero_strides_are_layout_valid():
    # an expanded (broadcast) tensor: all-zero strides except the unit last-dim stride
    lib = _lib()
    a = _bwd_args()
    for k in range(3):
        a.dout.stride[k] = 0
    assert lib.tda_validate_bwd(ctypes.byref(a)) == _abi.OK


@pytest.mark.parametrize("mutate,code", [
    (lambda a: setattr(a, "norms", None), _abi.ERR_NORMS),
    (lambda a: setattr(a, "workspace", None), _abi.ERR_WORKSPACE),
    (lambda a: setattr(a, "workspace_bytes", 8), _abi.ERR_WORKSPACE),
    (lambda a: setattr(a.dk2, "data", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a.dout, "data", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a, "head_dim", 32), _abi.ERR_HEAD_DIM),
])
def test_bwd_validator_rejects(mutate, code):
    lib = _lib()
    a = _bwd_args()
    mutate(a)
    assert lib.tda_validate_bwd(ctypes.byref(a)) == code
    assert lib.tda_bwd(ctypes.byref(a), None) == code


def test_bwd_norms_optional_without_normalize():
    lib = _lib()
    a = _bwd_args()
    a.normalize = 0
    a.norms = None
    assert lib.tda_validate_bwd(ctypes.byref(a)) == _abi.OK


def test_buffer_sizes():
    lib = _lib()
    assert lib.tda_occupancy_words(4, 16, 4096, 2) == 2 * 64 * 128 * 4
    assert lib.tda_occupancy_words(4, 16, 4096, 1) == 64 * 128 * 4
    assert lib.tda_occupancy_words(1, 1, 1, 1) == 1
    assert lib.tda_occupancy_words(1, 1, 33, 2) == 4
    # rectangular: query tiles x ceil(key tiles / 32) words per row
    assert lib.tda_occupancy_words_kv(1, 1, 33, 100, 2) == 2 * 2 * 1
    assert lib.tda_occupancy_words_kv(1, 1, 1, 5000, 1) == 1 * ((5000 + 31) // 32 + 31) // 32
    assert lib.tda_occupancy_words_kv(2, 3, 64, 64, 2) == lib.tda_occupancy_words(2, 3, 64, 2)
    assert lib.tda_norms_floats_kv(2, 3, 10, 20, 2) == 2 * 6 * 30
    assert lib.tda_norms_floats_kv(2, 3, 10, 10, 1) == lib.tda_norms_floats(2, 3, 10, 1)
    # one query tile: + the decode partials, [B*H][ceil(key tiles / 32)][Nq][128] floats
    assert lib.tda_fwd_workspace_bytes_kv(1, 1, 1, 5000, 1) == 256 + 5 * 1 * 128 * 4
    # more query tiles: + the candidate keys, per list 32 keys and a count, then a queue of query
    # tiles (a count block of 64 words and one item per head and query tile)
    r256 = lambda b: 256 * ((b + 255) // 256)  # noqa: E731
    cand = lambda lists, tiles: r256(lists * (1 + 32) * 4) + r256((64 + tiles) * 4)  # noqa: E731
    # + the int8 screen's keys (head_dim 128 bytes per row and branch) and their {scale, bound}
    k8 = lambda rows, d=128: r256(rows * d) + r256(rows * 8)  # noqa: E731
    assert lib.tda_fwd_workspace_bytes_kv(1, 1, 33, 5000, 1) == (256 * ((2 * 5 * 4 + 255) // 256) + cand(2, 2)
                                                              + k8(5000))
    assert lib.tda_occupancy_words_kv(1, 1, 33, 0, 2) == 0
    assert lib.tda_occupancy_words(1, 1, 33, 3) == 0
    assert lib.tda_norms_floats(4, 16, 4096, 2) == 4 * 64 * 4096
    assert lib.tda_norms_floats(1, 8, 128, 1) == 2 * 8 * 128
    # two branches: partial pairs and one dk weight per pair-list slot (32), then a key-tile
    # queue (a count block of 64 words and one item per pair-list slot)
    lists = 2 * 64 * 128
    assert lib.tda_bwd_workspace_bytes(4, 16, 4096, 128) == (lists * (2 + 32) + 64 + lists * 32) * 4
    # bitmask scratch, rounded up to 256 bytes, then the candidate lists
    assert lib.tda_fwd_workspace_bytes(4, 16, 4096, 2) == (2 * 64 * 128 * 4 * 4 + cand(2 * 64 * 128, 64 * 128)
                                                           + k8(2 * 64 * 4096))
    assert lib.tda_fwd_workspace_bytes(1, 1, 33, 1) == 256 + cand(2, 2) + k8(33)
    assert lib.tda_fwd_workspace_bytes(1, 1, 33, 3) == 0
    assert lib.tda_occupancy_words(0, 1, 1, 1) == 0


def test_error_strings():
    lib = _lib()
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11, -100):
        s = lib.tda_error_string(code).decode()
        assert s and s != "unknown error", code
    assert lib.tda_error_string(-55).decode() == "unknown error"


# ------------------------------------------------------------- Python boundary
def test_cpu_tensors_rejected_no_fallback():
    from tda_amd import differential_threshold_rela_triton, threshold_rela_triton
    x = torch.randn(1, 1, 8, 64)
    with pytest.raises(ValueError, match="GPU only"):
        threshold_rela_triton(x, x, x, 1.0)
    with pytest.raises(ValueError, match="GPU only"):
        differential_threshold_rela_triton(x, x, x, x, x, 1.0, 0.5)


def test_shape_mismatch_rejected():
    from tda_amd import threshold_rela_triton
    with pytest.raises(ValueError, match="shape mismatch"):
        threshold_rela_triton(torch.randn(1, 1, 8, 64), torch.randn(1, 1, 9, 64), torch.randn(1, 1, 8, 64), 1.0)
    with pytest.raises(ValueError, match="batch, heads, seq_len, head_dim"):
        threshold_rela_triton(torch.randn(8, 64), torch.randn(8, 64), torch.randn(8, 64), 1.0)


def test_missing_library_is_a_clear_error(tmp_path):
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _abi.load(str(tmp_path / "nope.so"))


def test_error_code_mapping():
    _lib()
    with pytest.raises(ValueError, match="head_dim"):
        _abi.check(_abi.ERR_HEAD_DIM, "tda_fwd")
    with pytest.raises(RuntimeError, match="launch failed"):
        _abi.check(_abi.ERR_HIP, "tda_fwd")
    _abi.check(_abi.OK, "tda_fwd")


@pytest.mark.parametrize("mutate,code", [
    (lambda a: setattr(a, "abi_version", 99), _abi.ERR_ABI),
    (lambda a: setattr(a, "head_dim", 96), _abi.ERR_HEAD_DIM),
    (lambda a: setattr(a, "beta", None), _abi.ERR_NULL_POINTER),
    (lambda a: setattr(a.q1, "data", FAKE + 2), _abi.ERR_LAYOUT),
    (lambda a: setattr(a, "norms", None), _abi.ERR_NORMS),
    (lambda a: setattr(a, "q_offset", -1), _abi.ERR_OFFSET),
    # its workspace is the library's own: the caller's workspace fields are not read
    (lambda a: setattr(a, "workspace", None), _abi.OK),
])
def test_fwd_noalloc_validates_like_tda_fwd(mutate, code):
    lib = _lib()
    a = _fwd_args()
    mutate(a)
    if code == _abi.OK:
        a.head_dim = 100  # stop at the validator anyway: no GPU here
        assert lib.tda_fwd_noalloc(ctypes.byref(a), None) == _abi.ERR_HEAD_DIM
    else:
        assert lib.tda_fwd_noalloc(ctypes.byref(a), None) == code


def test_fwd_noalloc_rejects_workspace_beyond_its_array():
    """A call needing more workspace than TDA_NOALLOC_SCRATCH_BYTES fails with ERR_SCRATCH
    before touching a GPU; the limit in the header matches the binding's."""
    lib = _lib()
    assert f"TDA_NOALLOC_SCRATCH_BYTES ((size_t){_abi.NOALLOC_SCRATCH_BYTES >> 20} << 20)" in open(HEADER).read()
    shape = (8, 64, 8192, 128)
    assert lib.tda_fwd_workspace_bytes(*shape[:3], 2) > _abi.NOALLOC_SCRATCH_BYTES
    a = _fwd_args(shape)
    assert lib.tda_fwd_noalloc(ctypes.byref(a), None) == _abi.ERR_SCRATCH
    assert b"16 MiB" in lib.tda_error_string(_abi.ERR_SCRATCH)


def test_launch_timing_arming_without_a_device():
    """tda_time_next_call only records the caller's events: NULL events with n > 0 are an
    error, n = 0 disarms, and a thread that made no timed call reports no launches."""
    lib = _lib()
    assert lib.tda_time_next_call(None, 3) == _abi.ERR_NULL_POINTER
    assert lib.tda_time_next_call(None, 0) == _abi.OK
    assert lib.tda_timed_launches() == 0
    assert lib.tda_timed_launch_name(0) is None
    assert lib.tda_timed_launch_name(-1) is None
    # an armed call that fails validation records nothing and stays armed for the next one
    evs = (ctypes.c_void_p * 2)(None, None)
    assert lib.tda_time_next_call(evs, 2) == _abi.OK
    assert lib.tda_fwd(None, None) == _abi.ERR_NULL_POINTER
    assert lib.tda_timed_launches() == 0
    assert lib.tda_time_next_call(None, 0) == _abi.OK
