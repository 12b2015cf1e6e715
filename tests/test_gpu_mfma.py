"""The device re-check of the MFMA fixture: v_mfma_f32_16x16x32_bf16 on this MI355X gives, bit for
bit, the outputs tests/golden/mfma_bf16_16x16x32.npz recorded (whose model, the oracle's
or_mfma_dot32, tests/test_mfma_model.py pins on the CPU), through the probe library's one-instruction
kernel (fx_probe.hip, fxp_mfma)."""
import os
import sys

import numpy as np
import pytest

FIX = os.path.join(os.path.dirname(__file__), "golden", "mfma_bf16_16x16x32.npz")


@pytest.mark.gpu
def test_instruction_matches_the_fixture(rt):
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_mfma_fixture as M
    z = np.load(FIX)
    print(f"[mfma] {z['A'].shape[0]} instructions", flush=True)
    D = M.run(M.probe_lib(), z["A"], z["B"], z["C"])
    bad = D.view(np.uint32) != z["D"].view(np.uint32)
    assert not bad.any(), (int(bad.sum()), np.argwhere(bad)[:4].tolist())
