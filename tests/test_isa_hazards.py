"""The kernels' gfx950 assembly has no MFMA result used too early on any control-flow path.

The hardware does not interlock VALU or store uses of a VGPR written by an MFMA; the
compiler inserts the wait states, and was seen to miss them on a branch path (a threshold
test reading scores 7 wait states after the MFMA, which made the screen drop tiles at
random).  tda_amd.isa_check compiles every kernel source to assembly and walks every path.
CPU only (hipcc cross-compiles); the synthetic snippets pin the scanner itself."""
import os

import pytest

from tda_amd import build, isa_check

HAS_HIPCC = os.path.exists(build.HIPCC)


def _kernel(body: str) -> str:
    return "_Z1kv:\n" + body + "\n\ts_endpgm\n"


def test_scanner_flags_a_read_on_a_branch_path():
    asm = _kernel("""
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\ts_cmp_gt_i32 s8, s9
\ts_cbranch_scc1 .LBB0_2
\ts_nop 7
\ts_nop 7
.LBB0_2:
\tv_max_f32_e32 v30, v3, v3""")
    hz = isa_check.scan(asm)["_Z1kv"]
    assert [(ws, kind) for ws, kind, *_ in hz] == [(2, "read")]  # s_cmp, s_cbranch; fall-through waits 18


def test_scanner_accepts_enough_wait_states_and_checks_each_kind():
    ok = _kernel("""
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\ts_nop 7
\ts_nop 3
\tv_max_f32_e32 v30, v3, v3
\tds_write_b128 v40, v[0:3]""")
    assert isa_check.scan(ok) == {}
    bad = _kernel("""
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\tds_write_b128 v40, v[0:3]
\tv_mov_b32_e32 v5, 0
\tv_mfma_f32_32x32x16_bf16 v[32:47], v[12:15], v[20:23], v[32:47]""")
    kinds = sorted(kind for _, kind, *_ in isa_check.scan(bad)["_Z1kv"])
    assert kinds == ["WAW", "read", "srcAB"]
    # the 16-pass fp32 MFMA needs 20 wait states: 12 are not enough
    f32 = _kernel("""
\tv_mfma_f32_32x32x2f32 v[0:15], v16, v17, v[0:15]
\ts_nop 7
\ts_nop 3
\tv_max_f32_e32 v30, v3, v3""")
    assert isa_check.scan(f32)


def test_scanner_skips_exec_zero_edges_only_while_exec_is_unchanged():
    skip = _kernel("""
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\ts_cbranch_execz .LBB0_2
\ts_nop 7
\ts_nop 7
.LBB0_2:
\tv_mov_b32_e32 v3, 0""")
    assert isa_check.scan(skip) == {}
    follow = _kernel("""
\tv_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]
\ts_and_saveexec_b64 s[0:1], vcc
\ts_cbranch_execz .LBB0_2
\ts_nop 7
\ts_nop 7
.LBB0_2:
\ts_or_b64 exec, exec, s[0:1]
\tv_mov_b32_e32 v3, 0""")
    assert isa_check.scan(follow)


@pytest.mark.skipif(not HAS_HIPCC, reason="hipcc not available")
def test_kernels_have_no_mfma_result_hazards():
    res = isa_check.check_all()
    msg = "; ".join(f"{src}:{k}:{h[0][:2]}" for src, ks in res.items() for k, h in ks.items())
    assert res == {}, msg
