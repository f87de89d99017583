"""Wait states after buffer stores, checked in the generated gfx950 assembly.

A VALU write to the data registers of a 12- or 16-byte buffer store in the
cycles right after the store can reach memory in the store's place.  The
compiler inserts wait states there only when the store's offset operand is a
constant, not when it is an SGPR; on gfx950 such a write, one instruction
after `buffer_store_dwordx4 ..., s67 offen`, replaced the first dword of ~2%
of the GRPO step's gradient vectors.  Every buffer store in the kernels goes
through a helper that adds `s_nop 1` (two wait states); this test compiles
each source that issues buffer stores and checks, for every such store in
every kernel, that no VALU instruction writes one of its data registers
before two wait states have passed.  Stores are found by walking the listing
in order (a branch target inside the window is walked through, which only
makes the check stricter).
"""
from __future__ import annotations

import os
import re

import pytest

import isa_listing

CSRC = isa_listing.CSRC
WAIT_STATES = 2

STORE = re.compile(r"buffer_store_dwordx[34] v\[(\d+):(\d+)\]")
VALU_DST = re.compile(r"v_\S+\s+v(?:\[(\d+):(\d+)\]|(\d+))\b")
NOP = re.compile(r"s_nop (\d+)")


def _sources_with_buffer_stores():
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith(".hip"):
            with open(os.path.join(CSRC, name)) as f:
                if "raw_buffer_store" in f.read():
                    out.append(name)
    return out


def _instructions(listing: str):
    """(kernel, instruction) pairs of a device assembly listing, comments,
    directives and labels dropped."""
    kernel = None
    for line in listing.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel = m.group(1)
            continue
        s = line.split(";")[0].strip()
        if not s or s.startswith(".") or s.endswith(":") or kernel is None:
            continue
        yield kernel, s


def hazards(listing: str):
    """Buffer stores followed, within WAIT_STATES wait states, by a VALU
    write to one of their data registers: [(kernel, store, writer)]."""
    ins = list(_instructions(listing))
    found = []
    for i, (kernel, s) in enumerate(ins):
        m = STORE.match(s)
        if not m:
            continue
        lo, hi = int(m.group(1)), int(m.group(2))
        waited = 0
        for k2, nxt in ins[i + 1:]:
            if k2 != kernel or waited >= WAIT_STATES:
                break
            n = NOP.match(nxt)
            if n:
                waited += int(n.group(1)) + 1
                continue
            d = VALU_DST.match(nxt)
            if d:
                a = int(d.group(1) or d.group(3))
                b = int(d.group(2) or d.group(3))
                if not (b < lo or a > hi):
                    found.append((kernel, s, nxt))
                    break
            waited += 1
    return found


def test_detector_flags_the_pattern_that_failed():
    """The check itself: the sequence from the failing build is flagged, the
    same with `s_nop 1` in between is not, nor a write to other registers."""
    bad = "_Zk:\n\tbuffer_store_dwordx4 v[58:61], v1, s[76:79], s67 offen nt\n" \
          "\tv_lshlrev_b32_e32 v58, 16, v54\n"
    good = "_Zk:\n\tbuffer_store_dwordx4 v[58:61], v1, s[76:79], s67 offen nt\n" \
           "\ts_nop 1\n\tv_lshlrev_b32_e32 v58, 16, v54\n"
    other = "_Zk:\n\tbuffer_store_dwordx4 v[58:61], v1, s[76:79], s67 offen nt\n" \
            "\tv_lshlrev_b32_e32 v62, 16, v54\n"
    late = "_Zk:\n\tbuffer_store_dwordx4 v[58:61], v1, s[76:79], s67 offen nt\n" \
           "\tv_add_f32_e32 v2, v3, v4\n\tv_mov_b32_e32 v60, 0\n"
    assert len(hazards(bad)) == 1
    assert hazards(good) == [] and hazards(other) == []
    assert len(hazards(late)) == 1  # one wait state passed, two are needed


@pytest.mark.skipif(not isa_listing.available(), reason="hipcc not available")
@pytest.mark.parametrize("source", _sources_with_buffer_stores())
def test_buffer_stores_have_wait_states(source):
    listing = isa_listing.listing(source)
    n_stores = len(STORE.findall(listing))
    assert n_stores > 0, f"{source}: no buffer stores in the listing"
    found = hazards(listing)
    assert not found, (f"{source}: {len(found)} of {n_stores} buffer stores are followed by a "
                       f"VALU write of their data registers within {WAIT_STATES} wait states, "
                       f"e.g. {found[0]}")
