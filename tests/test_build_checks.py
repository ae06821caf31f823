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
