"""CPU checks of the build's assembly checks: the 4x4x4 MFMA chains of
qmv_b4.hip are inline assembly, so mlxcel_amd.build.check_b4_mfma_chains
guards their register ties and wait states.  A well-formed chain passes and
each planted mistake is caught; the built library's own assembly (when
present) passes."""
import os

import pytest

from mlxcel_amd import build as B

GOOD = """\
kernel:
\tv_perm_b32 v45, s0, v3, v45
\t;;#ASMSTART
\ts_nop 1
\tv_mfma_f32_4x4x4_16b_bf16 v[2:5], v[30:31], v[12:13], 0
\t;;#ASMEND
\tv_fma_f32 v7, v29, v26, 0
\ts_nop 1
\tv_mfma_f32_4x4x4_16b_bf16 v[2:5], v[14:15], v[32:33], v[2:5]
\ts_nop 0
\ts_nop 7
\ts_nop 7
\tv_fmac_f32_e32 v7, v28, v3
\ts_endpgm
"""


def test_good_chain_passes():
    assert B.check_b4_mfma_chains(GOOD) == 2


@pytest.mark.parametrize("old,new,msg", [
    ("v[2:5], v[30:31], v[12:13], 0", "v[2:5], v[4:5], v[12:13], 0", "overlaps"),
    ("v[32:33], v[2:5]", "v[32:33], v[6:9]", "neither 0 nor|wait states"),
    ("\ts_nop 1\n\tv_mfma_f32_4x4x4_16b_bf16 v[2:5], v[14:15]", "\tv_mfma_f32_4x4x4_16b_bf16 v[2:5], v[14:15]",
     "not s_nop"),
    ("\ts_nop 7\n\ts_nop 7\n", "\ts_nop 7\n", "wait states"),
    ("\ts_nop 7\n\ts_nop 7\n\tv_fmac", "\ts_cbranch_scc1 .LBB0_2\n\ts_nop 7\n\ts_nop 7\n\tv_fmac", "wait states"),
])
def test_planted_mistakes_are_caught(old, new, msg):
    bad = GOOD.replace(old, new, 1)
    assert bad != GOOD
    with pytest.raises(RuntimeError, match=msg):
        B.check_b4_mfma_chains(bad)


def test_no_mfma_is_an_error():
    with pytest.raises(RuntimeError, match="no 4x4x4 MFMA"):
        B.check_b4_mfma_chains("kernel:\n\ts_endpgm\n")


@pytest.mark.skipif(not os.path.exists(B.B4_ASM), reason="library not built here (no qmv_b4 assembly)")
def test_built_assembly_passes():
    assert B.check_b4_mfma_chains(open(B.B4_ASM).read()) > 0
