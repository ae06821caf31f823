"""(batch, head) pairs of config 3 ([4, 32, 2048, 128]) that the full-size
tests check against the oracle.  The prefill kernels deal
bh = batch * 32 + head to XCD bh % 8, slot (bh / 8) % 4 of a four-head group,
group bh / 32 (sdpa_flash_bf16_pipe.hip, block mapping): these eight cover
every XCD residue, every group slot twice and every group twice."""
CONFIG3_BH = [0, 9, 50, 59, 68, 77, 118, 127]
CONFIG3_HEADS = [(bh // 32, bh % 32) for bh in CONFIG3_BH]
