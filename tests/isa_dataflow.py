"""Reads of vector registers that no write reaches, found in gfx950 device
assembly.

A kernel starts with only v0 written (the packed work-item ids); any other
VGPR holds whatever the previous wave on that SIMD left there.  This module
builds each kernel's control-flow graph from the listing (labels, s_branch,
s_cbranch_*, s_endpgm), runs a must-be-written dataflow over it (a register
counts as written at a block's entry only when it is written on every path
from the kernel's entry) and reports each instruction that reads a register
that some path leaves unwritten.

Conventions of the compiler's output that the analysis follows:
  * ``; implicit-def: $vgprN...`` comments mark values the compiler leaves
    undefined on purpose because nothing reads them on that path; they count
    as writes.
  * ``v_mad_u64_u32 / v_mad_i64_i32 vD[2], s, a, b, vC[2]`` with the high
    half of the addend unwritten is the compiler's 64 x 32-bit multiply: only
    the high half of the result depends on it, so that half stays unwritten
    and is reported only if something reads it.
A write under a partial exec mask counts as a write of the whole register;
this makes the check weaker, never noisier.
"""
from __future__ import annotations

import re

_REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_IMPLICIT = re.compile(r"implicit-def: (.*)")
_IMPLICIT_V = re.compile(r"vgpr(\d+)")
_LABEL = re.compile(r"^(\.LBB\w+):")
_BB = re.compile(r"^; %bb\.\d+:")
_BRANCH = re.compile(r"^s_(branch|cbranch_\w+|endpgm)\b\s*(\S*)")
_NO_VDST = ("global_store", "buffer_store", "ds_write", "ds_store", "flat_store",
            "scratch_store", "v_cmp", "v_readlane", "v_readfirstlane", "s_")
_READS_VDST = ("v_fmac", "v_mac", "v_writelane", "v_dot2c", "v_pk_fmac")
_MAD64 = ("v_mad_u64_u32", "v_mad_i64_i32")


def _mask(tok: str) -> int:
    m = 0
    for g in _REG.finditer(tok):
        if g.group(3) is not None:
            m |= 1 << int(g.group(3))
        else:
            for r in range(int(g.group(1)), int(g.group(2)) + 1):
                m |= 1 << r
    return m


def _operands(text: str) -> list[str]:
    ops, depth, cur = [], 0, ""
    for ch in text:
        depth += (ch == "[") - (ch == "]")
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return ops


def _effect(ins: str):
    """(reads, writes, addend_hi, result_hi) bit masks of one instruction;
    the last two are nonzero only for a 64-bit multiply-add."""
    parts = ins.split(None, 1)
    op, rest = parts[0], (parts[1] if len(parts) > 1 else "")
    ops = _operands(rest)
    if not ops:
        return 0, 0, 0, 0
    every = 0
    for o in ops:
        every |= _mask(o)
    no_vdst = (op.startswith(_NO_VDST) or op.endswith("_lds") or re.search(r"\blds\b", rest)
               or ("atomic" in op and not re.search(r"\b(glc|sc0)\b", rest))
               or (op.startswith("ds_")
                   and not re.match(r"ds_(read|load|bpermute|permute|swizzle|\w*rtn)", op)))
    if no_vdst:
        if op.startswith(("v_cmp", "v_readlane", "v_readfirstlane")):
            every &= ~_mask(ops[0])
        return every, 0, 0, 0
    dst = _mask(ops[0])
    reads = 0
    for o in ops[1:]:
        reads |= _mask(o)
    if op.startswith(_READS_VDST) or "d16" in op:
        reads |= dst
    if op.startswith(_MAD64) and len(ops) == 5:
        g = re.fullmatch(r"v\[(\d+):(\d+)\]", ops[4])
        d = re.fullmatch(r"v\[(\d+):(\d+)\]", ops[0])
        if g and d:
            hi = 1 << int(g.group(2))
            return reads & ~hi, dst, hi, 1 << int(d.group(2))
    return reads, dst, 0, 0


def _blocks(lines: list[str]):
    blocks, labels, cur = [], {}, []
    for raw in lines:
        s = raw.strip()
        lab = _LABEL.match(s)
        if lab or _BB.match(s):
            if cur:
                blocks.append(cur)
            cur = []
            if lab:
                labels[lab.group(1)] = len(blocks)
            continue
        if not s:
            continue
        cur.append(s)
        if _BRANCH.match(s):
            blocks.append(cur)
            cur = []
    if cur:
        blocks.append(cur)
    succ = []
    for i, b in enumerate(blocks):
        code = [x for x in b if not x.startswith((";", "."))]
        m = _BRANCH.match(code[-1]) if code else None
        nxt = [i + 1] if i + 1 < len(blocks) else []
        if m is None:
            succ.append(nxt)
        elif m.group(1) == "endpgm":
            succ.append([])
        elif m.group(1) == "branch":
            succ.append([labels[m.group(2)]])
        else:
            succ.append([labels[m.group(2)]] + nxt)
    return blocks, succ


def _compile_block(block: list[str]):
    steps = []
    for s in block:
        m = _IMPLICIT.search(s)
        if m:
            w = 0
            for r in _IMPLICIT_V.findall(m.group(1)):
                w |= 1 << int(r)
            steps.append((0, w, 0, 0, s))
            continue
        if s.startswith((";", ".")):
            continue
        steps.append((*_effect(s.split(";")[0].strip()), s))
    return steps


def _run(steps, written: int, report=None) -> int:
    for reads, writes, add_hi, res_hi, text in steps:
        missing = reads & ~written
        if missing and report is not None:
            report.append((text, [r for r in range(512) if missing >> r & 1]))
        addend_hi_written = bool(written & add_hi)
        written |= writes
        if add_hi and not addend_hi_written:
            written &= ~res_hi
    return written


def undefined_reads_of_kernel(lines: list[str]):
    """[(instruction, [registers])] for one kernel's body."""
    blocks, succ = _blocks(lines)
    if not blocks:
        return []
    steps = [_compile_block(b) for b in blocks]
    entry = [None] * len(blocks)
    entry[0] = 1  # v0
    work = [0]
    while work:
        i = work.pop()
        out = _run(steps[i], entry[i])
        for j in succ[i]:
            new = out if entry[j] is None else entry[j] & out
            if new != entry[j]:
                entry[j] = new
                work.append(j)
    report = []
    for i, e in enumerate(entry):
        if e is not None:
            _run(steps[i], e, report)
    return report


def kernels(listing: str) -> dict[str, list[str]]:
    """Kernel name -> body lines, for the symbols the listing declares with
    .amdhsa_kernel."""
    names = set(re.findall(r"^\s*\.amdhsa_kernel (\S+)", listing, re.M))
    out, name, body = {}, None, []
    for line in listing.splitlines():
        m = re.match(r"^(\S+):", line)
        if m and m.group(1) in names:
            name, body = m.group(1), []
            continue
        if name is not None:
            if line.startswith(".Lfunc_end"):
                out[name] = body
                name = None
            else:
                body.append(line)
    return out


def undefined_reads(listing: str):
    """{kernel: [(instruction, [registers])]} for every kernel of a listing
    that reads a VGPR some path leaves unwritten."""
    found = {}
    for name, body in kernels(listing).items():
        rep = undefined_reads_of_kernel(body)
        if rep:
            found[name] = rep
    return found
