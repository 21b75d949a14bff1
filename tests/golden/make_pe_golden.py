"""Writes tests/golden/pe_transforms.npz: input / output vectors of the reference's own positional-
encoding modules, evaluated by torch on the CPU.

The oracle's restatement of these transforms (oracle/pe_oracle.py: pope_transform, rope_rotate,
fope_effective_freqs, yarn_inv_freq) is pinned by closed forms to tolerance level; what closed forms
leave open is the bit pattern torch-CPU gives for the reference's own sequence of pow, outer, add,
cos, sin and softplus.  These vectors hold that bit pattern for small cases of

* PoPEEmbedding.forward_query / forward_key (src/model/pope.py:124-183), plain and floor-clipped,
  start_pos 0 and past the cached table (the on-the-fly extension branch, :99-104);
* FoPEPoPEEmbedding.forward_query / forward_key (src/model/fpope.py:266-338) in fp32;
* RotaryEmbedding / NTKAwareRotaryEmbedding / YaRNRotaryEmbedding.forward (src/model/rope.py).

Run only in the build container, which holds /root/reference (the GPU box does not): each module
file is loaded on its own with importlib (no package __init__; they import only torch), its
parameters are drawn from a fixed seed, and the arrays are written with numpy.savez_compressed
(no pickles).

    python tests/golden/make_pe_golden.py
"""

import importlib.util
import os

import numpy as np
import torch

REF = "/root/reference/src/model"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "pe_transforms.npz")


def load(name):
    spec = importlib.util.spec_from_file_location("ref_" + name, os.path.join(REF, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    pope, fpope, rope = load("pope"), load("fpope"), load("rope")
    torch.manual_seed(20261202)
    out = {}
    B, S, H, Hkv, D = 1, 12, 2, 1, 16

    def inputs(tag, h=H, d=D):
        x = torch.randn(B, S, h, d) * 3.0  # spans softplus's linear region (threshold 20 excluded)
        out[tag] = x.numpy()
        return x

    with torch.no_grad():
        # PoPE: table of 64 positions; start 0, start 40 (inside), start 70 (past the table: the
        # on-the-fly branch); plain and floor-clipped at training length 64 (clips 11 of 16 dims)
        for floor in (False, True):
            m = pope.PoPEEmbedding(D, max_seq_len=64, training_length=64, use_floor=floor, delta_init="uniform")
            m.phase_bias.data[0] = 1.5      # exercises the key-side clamp at both ends
            m.phase_bias.data[1] = -7.0
            t = "pope_floor" if floor else "pope"
            out[t + "_eff_freqs"] = m.effective_freqs.numpy()
            out[t + "_phase_bias"] = m.phase_bias.detach().numpy()
            for start in (0, 40, 70):
                xq, xk = inputs(f"{t}_{start}_xq"), inputs(f"{t}_{start}_xk")
                out[f"{t}_{start}_q"] = m.forward_query(xq, start).numpy()
                out[f"{t}_{start}_k"] = m.forward_key(xk, start).numpy()

        # FoPE (fp32 inputs, so positions are fp32): 4 Fourier terms, normalised coefficients
        m = fpope.FoPEPoPEEmbedding(D, max_seq_len=64, num_fourier_terms=4, training_length=64, delta_init="uniform")
        out["fope_base_freqs"] = m.base_freqs.numpy()
        out["fope_coeffs"] = m.fourier_coeffs.detach().numpy()
        out["fope_indices"] = m.fourier_indices.numpy()
        out["fope_phase_bias"] = m.phase_bias.detach().numpy()
        for start in (0, 37):
            xq, xk = inputs(f"fope_{start}_xq"), inputs(f"fope_{start}_xk")
            out[f"fope_{start}_q"] = m.forward_query(xq, start).numpy()
            out[f"fope_{start}_k"] = m.forward_key(xk, start).numpy()

        # RoPE family, head width 16, queries of 2 heads and keys of 1
        mods = {"rope": rope.RotaryEmbedding(D, max_seq_len=64),
                "ntk": rope.NTKAwareRotaryEmbedding(D, max_seq_len=64, scale=4.0),
                "yarn": rope.YaRNRotaryEmbedding(D, max_seq_len=64, scale=4.0, original_max_seq_len=16)}
        for t, m in mods.items():
            for start in (0, 29):
                xq, xk = inputs(f"{t}_{start}_xq"), inputs(f"{t}_{start}_xk", h=Hkv)
                q, k = m(xq, xk, start)
                out[f"{t}_{start}_q"] = q.numpy()
                out[f"{t}_{start}_k"] = k.numpy()
        out["yarn_mscale"] = np.asarray(float(mods["yarn"].mscale), dtype=np.float32)
    np.savez_compressed(OUT, **{k: np.ascontiguousarray(v) for k, v in out.items()})
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
