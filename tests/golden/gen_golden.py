#!/usr/bin/env python3
"""Write layer-level golden vectors from the reference's own torch model.

The absolute semantics of the projection / short-conv / gate / norm / o_proj
composition (GatedDeltaNet2::forward, src/module.rs:224-495) are pinned by
no closed form or invariant, so this script imports the reference's pure-torch
transcription of the layer, `Gdn2Reference` in tests/gen_reference.py, and
reproduces the first N_CASES cases of its ref_data.bin recipe
(tests/gen_reference.py:180-218): torch.manual_seed(1337), construct the
layer, then per case x = randn(1, 2**(i%6) + (i%7), D) and y = layer(x).
42 cases cover every sequence length the recipe produces (T in 1..38).

Run in the build container only (the reference is not present where the
GPU tests run); the output, tests/golden/layer_d64_h4.npz, is committed:
weights in burn's [in, out] layout plus (x, y) pairs.  No reference source
is copied into the fixture.
"""
import importlib.util
import os
import sys

import numpy as np

REF = "/root/reference/tests/gen_reference.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layer_d64_h4.npz")
N_CASES = 42


def main():
    import torch

    spec = importlib.util.spec_from_file_location("gdn2_gen_reference", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # definitions only; main() is guarded

    torch.manual_seed(1337)
    layer = mod.Gdn2Reference()
    layer.eval()

    def t(x):
        return x.detach().cpu().contiguous().numpy().astype(np.float32)

    arrays = {
        "cfg": np.array([mod.D, mod.H, mod.HK, mod.HV, int(round(mod.EXPAND_V * 10)),
                         int(mod.USE_SHORT_CONV), int(mod.ALLOW_NEG_EIGVAL)], np.int32),
        "norm_eps": np.array([mod.EPS], np.float64),
        "q_proj": t(layer.q_proj.weight.t()),
        "k_proj": t(layer.k_proj.weight.t()),
        "v_proj": t(layer.v_proj.weight.t()),
        "f_proj_0": t(layer.f_proj[0].weight.t()),
        "f_proj_1": t(layer.f_proj[1].weight.t()),
        "b_proj": t(layer.b_proj.weight.t()),
        "w_proj": t(layer.w_proj.weight.t()),
        "g_proj_0": t(layer.g_proj[0].weight.t()),
        "g_proj_1": t(layer.g_proj[1].weight.t()),
        "g_proj_1_bias": t(layer.g_proj[1].bias),
        "a_log": t(layer.A_log),
        "dt_bias": t(layer.dt_bias),
        "o_norm_weight": t(layer.o_norm_w),
        "o_proj": t(layer.o_proj.weight.t()),
        "q_conv_w": t(layer.q_conv_w.reshape(mod.KD, 4)),
        "k_conv_w": t(layer.k_conv_w.reshape(mod.KD, 4)),
        "v_conv_w": t(layer.v_conv_w.reshape(mod.VD, 4)),
    }
    with torch.no_grad():
        for i in range(N_CASES):
            seq_len = 2 ** (i % 6) + (i % 7)
            x = torch.randn(1, seq_len, mod.D)
            y = layer.forward(x)
            arrays[f"x{i}"] = t(x)
            arrays[f"y{i}"] = t(y)
    arrays["n_cases"] = np.array([N_CASES], np.int32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {N_CASES} cases")


if __name__ == "__main__":
    sys.exit(main())
