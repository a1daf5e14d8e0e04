"""Host side of the 4-bit RaBitQ codebooks (no GPU): the magnitude-levels
and sign-codebook JSON files the reference ships (copied as data under
tests/golden/pariskv_codebooks/: codebooks/magnitude_levels_m8*.json and
turboquant/codebooks/codebook_d128_m8_Kr1_Kw256_rabitq_sign.json)."""
from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from zoomkv_revision_amd import rabitq4

CB = Path(__file__).parent / "golden" / "pariskv_codebooks"


def test_eight_level_file_loads_as_bf16():
    thr, ctr = rabitq4.magnitude_levels(CB / "magnitude_levels_m8_4bit.json", device="cpu")
    d = json.loads((CB / "magnitude_levels_m8_4bit.json").read_text())
    assert thr.dtype == ctr.dtype == torch.bfloat16 and thr.shape == (7,) and ctr.shape == (8,)
    assert torch.equal(thr, torch.tensor(d["thresholds"], dtype=torch.bfloat16))
    assert torch.equal(ctr, torch.tensor(d["centers"], dtype=torch.bfloat16))


def test_builtin_levels_are_the_file_levels_rounded():
    """PC:266-270 hard-codes the file's levels to 4 decimals: the centers are
    the same bf16 values, the thresholds within one bf16 unit (the first one
    differs: 0.0843 against 0.08421), so codes made with the file's levels
    can differ from the built-in ones only at that boundary."""
    d = json.loads((CB / "magnitude_levels_m8_4bit.json").read_text())
    thr, ctr = rabitq4.magnitude_levels(device="cpu")
    assert torch.equal(ctr, torch.tensor(d["centers"], dtype=torch.bfloat16))
    file_thr = torch.tensor(d["thresholds"], dtype=torch.bfloat16)
    diff = (thr.view(torch.int16).int() - file_thr.view(torch.int16).int()).abs()
    assert int(diff.max()) <= 1 and int((diff != 0).sum()) == 1 and int(diff[0]) == 1
    assert all(abs(a - b) < 1e-3 for a, b in zip(rabitq4.MAG_THRESHOLDS, d["thresholds"]))


def test_four_level_file_is_rejected():
    """magnitude_levels_m8.json holds 4 levels (2 bits): not a 4-bit codebook."""
    with pytest.raises(ValueError):
        rabitq4.magnitude_levels(CB / "magnitude_levels_m8.json", device="cpu")


def test_sign_codebook_file_matches_the_quantizer_geometry():
    """The reference's sign codebook: d = 128, m = 8, K_r = 1, K_omega = 256
    rows of +-1 (the configuration MultiDimBlockQuantizer checks)."""
    d = json.loads((CB / "codebook_d128_m8_Kr1_Kw256_rabitq_sign.json").read_text())
    cfg = d["config"]
    assert (cfg["d"], cfg["m"], cfg["K_r"], cfg["K_omega"]) == (128, 8, 1, 256)
    signs = torch.tensor(d["angular_signs"], dtype=torch.float32)
    assert signs.shape == (256, 8) and set(signs.unique().tolist()) <= {-1.0, 1.0}
