"""Host-side checks of the native build recipe (jax-mlx-plugin_amd/build.py)."""
import re
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "jax-mlx-plugin_amd"))
import build as native_build  # noqa: E402

REMARKS = """k.hip:1:1: remark: Function Name: kern_a [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark:     VGPRs: 250 [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark:     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark:     SGPRs Spill: 24 [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark:     VGPRs Spill: {spill} [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark: Function Name: kern_b [-Rpass-analysis=kernel-resource-usage]
k.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_no_spill_check_accepts_sgpr_spills_only():
    native_build._check_no_spill(Path("k.hip"), REMARKS.format(scratch=0, spill=0))


@pytest.mark.parametrize("scratch,spill", [(92, 34), (4, 0), (0, 1)])
def test_no_spill_check_names_the_spilling_kernel(scratch, spill):
    with pytest.raises(RuntimeError, match="kern_a"):
        native_build._check_no_spill(Path("k.hip"), REMARKS.format(scratch=scratch, spill=spill))


def test_async_asm_kernels_are_guarded():
    kdir = Path(native_build.__file__).parent / "csrc" / "kernels"
    pat = re.compile(r'asm\s+volatile\(\s*"ds_read|\bds_(b128|tr)<')
    users = {p.name for p in kdir.glob("*.hip") if pat.search(p.read_text())}
    assert "sdpa_flash_bf16_pipe.hip" in users
    assert users <= native_build.NO_SPILL_FILES, users - native_build.NO_SPILL_FILES


def _kernel(body: str) -> str:
    lines = [l.strip() for l in body.strip().splitlines()]
    text = "\n".join(l if l.startswith((".LBB", ";")) else "\t" + l for l in lines)
    return f"\t.text\n_Z4kernv:\n{text}\n\ts_endpgm\n.Lfunc_end0:\n"


LDS_WAIT_OK = {
    "waited": """
        ds_read_b64_tr_b16 v[4:5], v0 offset:128
        ds_read_b64_tr_b16 v[6:7], v0 offset:256
        s_waitcnt lgkmcnt(0)
        v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], a[0:15]""",
    "oldest_retired_first": """
        ds_read_b64_tr_b16 v[4:5], v0 offset:128
        ds_read_b64_tr_b16 v[6:7], v0 offset:256
        s_waitcnt lgkmcnt(1)
        v_add_f32_e32 v1, v4, v5""",
    "raw_encoding": """
        ds_read_b128 v[4:7], v0
        s_waitcnt 0xc07f
        v_add_f32_e32 v1, v4, v7""",
    "in_order_lds_overwrite": """
        ds_read_b128 v[4:7], v0
        ds_read_b128 v[4:7], v0 offset:64
        s_waitcnt lgkmcnt(0)
        v_add_f32_e32 v1, v4, v7""",
    "both_paths_wait": """
        ds_read_b128 v[4:7], v0
        s_cbranch_scc1 .LBB0_2
        s_waitcnt lgkmcnt(0)
        s_branch .LBB0_3
.LBB0_2:
        s_waitcnt lgkmcnt(0)
.LBB0_3:
        v_add_f32_e32 v1, v4, v1""",
    "loop_waits_before_use": """
        ds_read_b32 v4, v0
.LBB0_1:
        s_waitcnt lgkmcnt(0)
        v_add_f32_e32 v1, v4, v1
        ds_read_b32 v4, v0
        s_cbranch_scc1 .LBB0_1
        s_waitcnt lgkmcnt(0)""",
}

LDS_WAIT_BAD = {
    "no_wait": ("""
        ds_read_b64_tr_b16 v[4:5], v0
        v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], a[0:15]""", "v_mfma"),
    "wait_too_shallow": ("""
        ds_read_b64_tr_b16 v[4:5], v0 offset:128
        ds_read_b64_tr_b16 v[6:7], v0 offset:256
        s_waitcnt lgkmcnt(1)
        v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], a[0:15]""", "v_mfma"),
    "valu_overwrites_pending": ("""
        ds_read_b128 v[4:7], v0
        v_mov_b32_e32 v6, 0
        s_waitcnt lgkmcnt(0)""", "v_mov_b32_e32 v6"),
    "lds_address_from_pending": ("""
        ds_read_b32 v4, v0
        ds_read_b32 v5, v4
        s_waitcnt lgkmcnt(0)""", "ds_read_b32 v5"),
    "scalar_load_may_return_first": ("""
        s_load_dwordx2 s[0:1], s[4:5], 0x0
        ds_read_b128 v[4:7], v0
        s_waitcnt lgkmcnt(1)
        v_add_f32_e32 v1, v4, v1""", "v_add_f32"),
    "one_path_skips_wait": ("""
        ds_read_b128 v[4:7], v0
        s_cbranch_scc1 .LBB0_2
        s_waitcnt lgkmcnt(0)
.LBB0_2:
        v_add_f32_e32 v1, v4, v1""", "v_add_f32"),
    "back_edge_skips_wait": ("""
        s_waitcnt lgkmcnt(0)
.LBB0_1:
        v_add_f32_e32 v1, v4, v1
        ds_read_b32 v4, v0
        s_cbranch_scc1 .LBB0_1
        s_waitcnt lgkmcnt(0)""", "v_add_f32"),
}


@pytest.mark.parametrize("case", sorted(LDS_WAIT_OK))
def test_lds_wait_check_accepts(case):
    native_build._check_lds_waits(Path("k.hip"), _kernel(LDS_WAIT_OK[case]))


@pytest.mark.parametrize("case", sorted(LDS_WAIT_BAD))
def test_lds_wait_check_names_the_early_read(case):
    body, what = LDS_WAIT_BAD[case]
    with pytest.raises(RuntimeError, match=r"_Z4kernv: line \d+: " + re.escape(what)):
        native_build._check_lds_waits(Path("k.hip"), _kernel(body))


def test_lds_wait_check_runs_on_the_built_kernels():
    """The build writes each guarded file's device assembly beside its object
    and checks it; the built assembly holds the kernels and passes."""
    obj_dir = native_build.OBJ_DIR / "kernels"
    built = sorted(obj_dir.glob("*.s"))
    if not built:
        pytest.skip("native library not built here")
    assert {p.with_suffix(".hip").name for p in built} >= native_build.NO_SPILL_FILES
    for p in built:
        text = p.read_text()
        assert len(re.findall(r"^_Z\S+:", text, re.M)) > 0
        native_build._check_lds_waits(p, text)
    gemm = obj_dir / "gemm16.s"
    stripped = "\n".join(l for l in gemm.read_text().splitlines() if "lgkmcnt" not in l)
    with pytest.raises(RuntimeError, match="before their LDS data arrives"):
        native_build._check_lds_waits(gemm, stripped)
