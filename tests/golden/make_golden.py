"""Write the committed golden fixtures (tests/golden/*.npz, *.json).

Two kinds:
  * known answers the reference's own tests hold (src/ops/mod.rs):
    the scale-1/128 round trip (:577-597), softmax([1,2,3]) (:421-427) and the
    hand-computed gemv (:489-494) -> known_answers.json;
  * Q8 vectors computed by the oracle on fixed inputs: a slice of the cfg1
    GEMV (64 rows of the SmolLM2-135M gate shape, K = 576), a 4x64 and an
    8x128 Q8_0x4 case, with the quantized activation, the per-block i32
    dots and the f32 outputs -> q8_vectors.npz.

Inputs come from the reference tests' LCG (tests/backends.rs:41-51), so a
fixture is reproducible from its seed alone; the arrays are stored anyway.

Run from the repository root: python tests/golden/make_golden.py
"""

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def q8_case(name, storage, out_dim, in_dim, rows, w_seed, x_seed, scale=0.04):
    w = (O.lcg_fill(out_dim * in_dim, w_seed) * np.float32(scale)).reshape(out_dim, in_dim)
    x = (O.lcg_fill(rows * in_dim, x_seed) * np.float32(4.0)).reshape(rows, in_dim)
    m = O.Matrix(w, storage)
    xq = np.stack([O.quantize(x[r])[0] for r in range(rows)])
    xs = np.stack([O.quantize(x[r])[1] for r in range(rows)])
    xh = np.stack([O.quantize(x[r])[2] for r in range(rows)])
    out = {f"{name}.w": w, f"{name}.x": x, f"{name}.xq": xq, f"{name}.xs": xs, f"{name}.xh": xh,
           f"{name}.dots": m.block_dots(xq.ravel()), f"{name}.y": m.project_cpu(x),
           f"{name}.logits": m.logits_cpu(x[0])}
    if storage == "q8_0":
        q, s = m.q8_0_data()
        out[f"{name}.wq"], out[f"{name}.ws"] = q, s
    else:
        out[f"{name}.blocks"] = m.q8_0x4_blocks()
    return out


def main():
    arrays = {}
    arrays.update(q8_case("cfg1_slice", "q8_0", 64, 576, 1, 11, 12))
    arrays.update(q8_case("x4_4x64", "q8_0x4", 4, 64, 2, 21, 22))
    arrays.update(q8_case("x4_8x128", "q8_0x4", 8, 128, 3, 31, 32))
    np.savez_compressed(os.path.join(HERE, "q8_vectors.npz"), **arrays)

    step = np.float32(1.0 / 128.0)
    vals = [float(np.float32(127.0 if lane == 0 else lane - 16.0) * step) for _ in range(2) for lane in range(32)]
    kat = {
        "source": "reference src/ops/mod.rs tests",
        "q8_step_multiples": {"values": vals, "scale": float(step)},
        "softmax_1_2_3": {"input": [1.0, 2.0, 3.0], "want": [0.09003057, 0.24472847, 0.66524094], "tol": 1e-6},
        "gemv_hand": {"w": [[1, 2, 3], [4, 5, 6]], "x": [1, 1, 1], "want": [6.0, 15.0]},
    }
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(kat, f, indent=1)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
