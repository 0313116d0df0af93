"""The checks of the built device code: the wait states of the inline-assembly DPP
multiply-adds in the Mamba-1 backward, and the single rounding convention for float16 results.

`metal-kernelops_amd/isa_check.py` holds the checks; `build()` runs them on the built objects
and fails the build on a problem.  Here the checkers themselves are tested on small listings
(so that a regression of a checker cannot let bad code through), and the built objects are
checked again when they are present.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "metal-kernelops_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)

import isa_check  # noqa: E402

OBJ = os.path.join(PKG, "_build", "selscan.o")
LIB = os.path.join(PKG, "metal_kernelops", "_lib", "libmko.so")
FMAC = "v_fmac_f32_dpp v10, v4, v5 row_newbcast:3 row_mask:0xf bank_mask:0xf bound_ctrl:1"


def _listing(body):
    out = ["0000000000001000 <k>:"]
    for n, text in enumerate(body):
        out.append(f"\t{text:58s} // {0x1000 + 4 * n:012X}: 00000000")
    return out


def _bad(body):
    return bool(isa_check.problems(_listing(body))[1])


def test_checker_finds_an_unsettled_source():
    """The DPP source written one instruction before is reported; behind s_nop 1 or two other
    instructions it is not; a branch landing between write and read makes it unverifiable."""
    assert _bad(["v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", FMAC])
    assert not _bad(["v_mul_f32_e32 v4, v1, v2", "s_nop 1", FMAC])
    far = ["v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", "v_add_f32_e32 v8, v1, v2", FMAC]
    assert not _bad(far) and isa_check.problems(_listing(far))[0] == 1
    assert _bad(["s_branch 1 <k+0xc>", "v_mul_f32_e32 v4, v1, v2", "v_add_f32_e32 v7, v1, v2", FMAC])


def test_checker_covers_every_input_and_exec():
    """The multiplier and the tied accumulator need the same two wait states as the DPP
    source; both outputs of a lane swap count as writes; a loaded register too; and a
    v_cmpx (it writes EXEC) needs five."""
    pad = "v_add_f32_e32 v7, v1, v2"
    assert _bad(["v_mul_f32_e32 v5, v1, v2", pad, FMAC])  # multiplier
    assert _bad(["v_mov_b32_e32 v10, v1", pad, FMAC])  # accumulator
    assert _bad(["v_permlane32_swap_b32_e32 v9, v4", pad, FMAC])  # second output of a swap
    assert _bad(["v_permlane16_swap_b32_e32 v5, v9", FMAC])  # first output of a swap
    assert _bad(["v_lshlrev_b64 v[4:5], 1, v[0:1]", pad, FMAC])  # a register pair
    assert _bad(["ds_read_b32 v4, v2", pad, FMAC])  # a load's destination
    assert not _bad(["ds_write_b32 v4, v5", pad, FMAC])  # a store reads its operands
    assert _bad(["v_cmpx_gt_f32_e32 vcc, v1, v2", pad, pad, pad, pad, FMAC])  # EXEC, 4 wait states
    assert not _bad(["v_cmpx_gt_f32_e32 vcc, v1, v2", pad, pad, pad, pad, pad, FMAC])
    assert not _bad(["v_cmp_gt_f32_e32 vcc, v4, v5", FMAC])  # a compare into VCC writes no VGPR
    assert not _bad(["v_mul_f32_e32 v4, v1, v2", "s_nop 0", pad, FMAC])
    # a loop head three instructions before: settled VGPRs, and the paths into it (the fall-
    # through and the back branch) carry no v_cmpx; one that does is reported
    loop = ["s_nop 4", "s_waitcnt lgkmcnt(0)", pad, pad, FMAC, "s_cbranch_scc1 1 <k+0x4>"]
    assert not _bad(loop)
    assert _bad(["s_nop 4", "s_waitcnt lgkmcnt(0)", pad, pad, FMAC, "v_cmpx_gt_f32_e32 vcc, v1, v2",
                 "s_cbranch_scc1 1 <k+0x4>"])


def test_dpp_fmac_inputs_are_settled_in_the_built_object():
    """The object `build()` produced.  Where the library exists, its objects must be there to
    check: a missing object fails rather than skips."""
    if not os.path.exists(OBJ):
        if os.path.exists(LIB) and os.path.isdir(os.path.join(PKG, "_build")):
            pytest.fail(f"{LIB} exists but {OBJ} is missing: rebuild with __graft_entry__.build()")
        pytest.skip("selscan.o not built here (run __graft_entry__.build() first)")
    assert isa_check.check_object(OBJ) > 0


def test_f16_rounding_checker():
    """A mixed-precision multiply-add with a float16 result (one rounding of the exact product)
    is reported, with its function; one with an fp32 result, and fp32-to-float16 conversions,
    are not."""
    assert isa_check.f16_rounding_problems(_listing(["v_fma_mixlo_f16 v3, v1, v2, 0 op_sel_hi:[1,0,0]"])) == {"k": 1}
    assert isa_check.f16_rounding_problems(_listing(["v_fma_mixhi_f16 v3, v1, v2, v4"])) == {"k": 1}
    assert isa_check.f16_rounding_problems(_listing(["v_mad_mixlo_f16 v3, v1, v2, v4"])) == {"k": 1}
    assert isa_check.f16_rounding_problems(_listing(["v_fma_mix_f32 v3, v1, v2, v4 op_sel_hi:[1,0,0]",
                                                     "v_cvt_pk_f16_f32 v5, v6, v7", "v_cvt_f16_f32_e32 v8, v9"])) == {}


@pytest.mark.parametrize("name", ["ssd.o", "ssd_bwd.o", "selscan.o", "state_update.o", "conv1d.o", "gated_norm.o"])
def test_built_objects_round_float16_results_one_way(name):
    """Every fp32-to-float16 rounding in the built kernels is a conversion of a finished fp32
    value.  The SSD backward's dA / ddt_bias depend on it: the gate kernel's row sums gy . y~
    and the du kernels' column sums u . du cancel only when both take u = step x rounded the
    same way, and a fused single rounding in one of them left float16 dA errors of 1e-2."""
    obj = os.path.join(PKG, "_build", name)
    if not os.path.exists(obj):
        if os.path.exists(LIB):
            pytest.fail(f"{LIB} exists but {obj} does not: rebuild with build()")
        pytest.skip("library not built")
    isa_check.check_f16_rounding(obj)
