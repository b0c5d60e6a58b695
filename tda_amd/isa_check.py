"""Static check of the gfx950 assembly of the kernels for matrix-core result hazards.

On CDNA3/CDNA4 the hardware does not interlock a VALU (or LDS/memory store) use of a VGPR
written by an MFMA: the compiler must place enough independent instructions or s_nop wait
states between them (for v_mfma_f32_32x32x16_bf16 and v_mfma_i32_32x32x32_i8, 8-pass ops on
gfx950: 12; for the 16-pass v_mfma_f32_32x32x2f32: 20).  hipcc was seen to count them on the fall-through path
only, leaving a read 7 wait states after the MFMA on a branch path that skipped a block.
This module compiles each kernel source to assembly and walks every control-flow path from
each MFMA for that many wait states, reporting:
  read   an instruction other than an MFMA reading the MFMA's destination registers
         (VALU sources, LDS/memory store data),
  srcAB  an MFMA reading them as its A or B operand,
  WAW    a VALU instruction writing them.
Each instruction counts one wait state and s_nop N counts N + 1.  An s_cbranch_execz or
s_cbranch_execnz edge is not followed when no instruction between the MFMA and the branch
writes EXEC: the branch then tests the EXEC the MFMA ran under, which is never empty in
these whole-wave loops.

    python -m tda_amd.isa_check          # compile and scan every kernel source
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

from . import build as _build

STORES = ("ds_write", "ds_store", "global_store", "buffer_store", "flat_store", "global_atomic",
          "buffer_atomic", "flat_atomic", "ds_add", "ds_bpermute", "ds_permute")


def _regs(tok: str) -> set:
    tok = tok.strip()
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _split(ins: str):
    parts = ins.split(None, 1)
    return parts[0], ([o.strip() for o in parts[1].split(",")] if len(parts) > 1 else [])


def _functions(asm: str) -> dict:
    """{kernel symbol: [('label', name) | ('ins', text) | ('end', text)]}"""
    funcs, cur = {}, None
    for line in asm.splitlines():
        if re.match(r"^_Z\S*:", line):
            cur = line.split(":")[0]
            funcs[cur] = []
            continue
        if cur is None:
            continue
        s = line.split(";")[0].strip()
        if not s:
            continue
        if s.startswith("."):
            if re.match(r"^\.LBB\S*:", s):
                funcs[cur].append(("label", s[:-1]))
            continue
        if s.startswith("s_endpgm"):
            funcs[cur].append(("end", s))
            cur = None
            continue
        funcs[cur].append(("ins", s))
    return funcs


def _window(op: str) -> int:
    # 16-pass fp32 32x32x2: 20; 8-pass bf16 32x32x16 and int8 32x32x32: 12
    return 20 if op.endswith("x2f32") else 12


def scan_function(body: list) -> list:
    """Hazards of one kernel: (wait states, kind, mfma, use, branch path)."""
    labels = {x[1]: i for i, x in enumerate(body) if x[0] == "label"}
    found = []
    for i, (kind, text) in enumerate(body):
        if kind != "ins" or not text.startswith("v_mfma"):
            continue
        op, ops = _split(text)
        dst, limit = _regs(ops[0]), _window(op)
        stack, seen = [(i + 1, 0, (), False)], set()
        while stack:
            j, ws, path, exec_changed = stack.pop()
            if (j, ws, exec_changed) in seen or ws >= limit or j >= len(body):
                continue
            seen.add((j, ws, exec_changed))
            k2, t2 = body[j]
            if k2 == "label":
                stack.append((j + 1, ws, path, exec_changed))
                continue
            if k2 == "end":
                continue
            op2, o2 = _split(t2)
            hit = None
            if op2.startswith("v_mfma"):
                if len(o2) >= 3 and (_regs(o2[1]) | _regs(o2[2])) & dst:
                    hit = "srcAB"
                else:
                    continue  # the next MFMA (a chain step): hazards are checked from it
            elif op2.startswith(STORES) or op2.startswith("v_"):
                srcs = o2 if op2.startswith(STORES) else o2[1:]
                if set().union(*[_regs(x) for x in srcs]) & dst if srcs else False:
                    hit = "read"
                elif op2.startswith("v_") and o2 and _regs(o2[0]) & dst:
                    hit = "WAW"
            if hit:
                found.append((ws, hit, text, t2, path))
            writes_exec = bool(o2) and o2[0].startswith("exec") or "saveexec" in op2
            ex = exec_changed or writes_exec
            n = int(o2[0], 0) + 1 if op2 == "s_nop" else 1
            if op2.startswith("s_cbranch") or op2 == "s_branch":
                target = o2[0] if o2 else ""
                follow = not (op2 in ("s_cbranch_execz", "s_cbranch_execnz") and not ex)
                if target in labels and follow:
                    stack.append((labels[target], ws + 1, path + (target,), ex))
                if op2 == "s_branch":
                    continue
            stack.append((j + 1, ws + n, path, ex))
    return found


def scan(asm: str) -> dict:
    """{kernel symbol: hazards} for every kernel in one assembly file with a hazard."""
    out = {}
    for name, body in _functions(asm).items():
        h = scan_function(body)
        if h:
            out[name] = h
    return out


def compile_asm(src: str, outdir: str) -> str:
    """gfx950 device assembly of one kernel source, with the library's own flags."""
    out = os.path.join(outdir, os.path.basename(src) + ".s")
    flags = [f for f in _build.HIP_FLAGS if f != "-fPIC"]
    cmd = [_build.HIPCC, *flags, "--cuda-device-only", "-S", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stderr}")
    with open(out) as f:
        return f.read()


def check_all(sources=None) -> dict:
    """Compile every kernel source and scan it.  Returns {source: {kernel: hazards}}."""
    sources = sources or _build.HIP_SOURCES
    with tempfile.TemporaryDirectory() as d:
        paths = [os.path.join(_build.CSRC, s) for s in sources]
        with ThreadPoolExecutor(max_workers=min(len(paths), os.cpu_count() or 1)) as ex:
            asms = list(ex.map(lambda p: compile_asm(p, d), paths))
    return {s: r for s, r in ((s, scan(a)) for s, a in zip(sources, asms)) if r}


if __name__ == "__main__":
    res = check_all()
    for src, kernels in res.items():
        for name, hz in kernels.items():
            for ws, kind, mfma, use, path in hz[:3]:
                print(f"{src} {name}\n   {kind} after {ws} wait states via {path or 'fall-through'}\n"
                      f"   {mfma}\n   {use}")
    print("hazards:", sum(len(h) for k in res.values() for h in k.values()))
    sys.exit(1 if res else 0)
