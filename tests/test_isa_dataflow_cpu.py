"""No kernel reads a vector register that some path leaves unwritten
(gfx950 assembly of every source, checked by tests/isa_dataflow.py).

A register that no write reaches holds what the previous wave on the SIMD
left there.  The first form of the GRPO token-weights kernel (one kernel
body branching on the loss kind at run time, a signed 32-bit thread id
widened to the 64-bit loop index) compiled so that the fixed-scale branch
reached its loop with the high half of that index never written: on the
GPU some waves skipped their stores, and a negative leftover would have
sent them below the output.  The instruction and register of that listing
are the detector's own test below; the library test then checks every
kernel of every source.
"""
from __future__ import annotations

import os

import pytest

import isa_listing
from isa_dataflow import kernels, undefined_reads, undefined_reads_of_kernel


def _reads(text: str):
    return undefined_reads_of_kernel(text.strip("\n").splitlines())


def test_detector_flags_a_path_that_skips_the_write():
    """The shape of the failing listing: the branch that skips the block
    writing v1 reaches a 64-bit compare of v[0:1]."""
    skipped = """
; %bb.0:
	s_cmp_eq_u32 s7, 1
	s_cbranch_scc0 .LBB0_2
; %bb.1:
	v_mov_b32_e32 v1, 0
.LBB0_2:
	v_cmp_gt_i64_e32 vcc, s[12:13], v[0:1]
	s_endpgm
"""
    both = skipped.replace("\ts_cmp_eq_u32 s7, 1\n", "\tv_mov_b32_e32 v1, 0\n\ts_cmp_eq_u32 s7, 1\n")
    marked = skipped.replace("\ts_cbranch_scc0 .LBB0_2\n",
                             "\t; implicit-def: $vgpr1\n\ts_cbranch_scc0 .LBB0_2\n")
    assert _reads(skipped) == [("v_cmp_gt_i64_e32 vcc, s[12:13], v[0:1]", [1])]
    assert _reads(both) == []
    assert _reads(marked) == []


def test_detector_follows_loops_and_stores():
    """A loop whose header reads a register written only inside the body
    is flagged (the first trip reads it unwritten); a store's data and
    address registers are reads."""
    loop = """
; %bb.0:
	v_mov_b32_e32 v2, 0
.LBB0_1:
	v_add_u32_e32 v2, v3, v2
	v_mov_b32_e32 v3, 1
	s_cbranch_scc0 .LBB0_1
; %bb.2:
	s_endpgm
"""
    store = """
; %bb.0:
	v_mov_b32_e32 v2, 0
	global_store_dword v[2:3], v4, off
	s_endpgm
"""
    assert _reads(loop) == [("v_add_u32_e32 v2, v3, v2", [3])]
    assert _reads(store) == [("global_store_dword v[2:3], v4, off", [3, 4])]


def test_detector_multiply_add_high_half():
    """The compiler's 64 x 32-bit multiply leaves the addend's high half
    unwritten; only a later read of the result's high half is a fault."""
    mad = """
; %bb.0:
	v_mov_b32_e32 v2, 7
	v_mov_b32_e32 v10, 0
	v_mad_u64_u32 v[10:11], s[8:9], s7, v2, v[10:11]
	v_mov_b32_e32 v9, v10
	v_mov_b32_e32 v11, 0
	v_add_u32_e32 v12, v11, v9
	s_endpgm
"""
    read_hi = mad.replace("\tv_mov_b32_e32 v11, 0\n", "")
    assert _reads(mad) == []
    assert _reads(read_hi) == [("v_add_u32_e32 v12, v11, v9", [11])]


@pytest.mark.skipif(not isa_listing.available(), reason="hipcc not available")
@pytest.mark.parametrize("source", isa_listing.sources())
def test_no_kernel_reads_an_unwritten_vgpr(source):
    text = isa_listing.listing(source)
    with open(os.path.join(isa_listing.CSRC, source)) as f:
        declares_kernels = "__global__" in f.read()
    found_kernels = kernels(text)
    assert bool(found_kernels) == declares_kernels, f"{source}: kernels not found in the listing"
    for name, body in found_kernels.items():
        assert not any("s_swappc" in line or "s_setpc" in line for line in body), \
            f"{source}: {name} calls a function (the check follows one kernel body)"
    found = undefined_reads(text)
    assert not found, "\n".join(
        f"{source}: {name}: {reads[:4]}" for name, reads in found.items())
