"""Writes the golden fixtures under tests/golden/ from third-party libraries (torch, numpy).

These vectors are produced without the oracle, so the oracle's decoders and conversions are checked
against an independent implementation:
  - e4m3fn.json : torch.float8_e4m3fn decode of all 256 bytes, and torch's float32 -> e4m3fn rounding
  - convert.json : torch's float32 -> bfloat16 / float16 rounding of edge values
  - gelu.json    : torch.nn.functional.gelu(approximate="tanh") in float64 on edge and random inputs
  - rmsnorm.json : torch.nn.functional.rms_norm in float64 with weight (offset + w) * (1 + scale), plus shift:
                   the RMSNorm of src/kernels/rmsnorm.ts:42-45, with and without the Krea modulation
torch-randn.json is the reference's own fixture (tests/fixtures/torch-randn.json), copied as data.

Run: python tests/golden/make_golden.py   (needs torch; the tests only read the JSON files)
"""
import json
import math
import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent


def f32_bits(v):
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def main():
    codes = torch.arange(256, dtype=torch.uint8)
    dec = codes.view(torch.float8_e4m3fn).to(torch.float64).tolist()
    table = ["nan" if math.isnan(v) else repr(v) for v in dec]
    neg_zero = [b for b in range(256) if dec[b] == 0.0 and math.copysign(1.0, dec[b]) < 0]
    (HERE / "e4m3fn.json").write_text(
        json.dumps({"source": f"torch {torch.__version__} float8_e4m3fn", "decode": table, "negative_zero": neg_zero},
                   indent=1))

    edge = [0.0, -0.0, 1.0, -2.0, 3.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, 1.0 + 2 ** -9, 65504.0, 65519.0, 65520.0,
            1e-8, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14, 2 ** -14 - 2 ** -25, 5.960464477539063e-08, 1e30, -1e-30,
            float("inf"), float("-inf"), 0.1, -0.3, 123.456, 3.3895313892515355e38, 1.1754943508222875e-38]
    rng = np.random.default_rng(5)
    rand = (rng.standard_normal(200) * np.exp(rng.uniform(-30, 30, 200))).astype(np.float32).tolist()
    vals = [float(np.float32(v)) for v in edge + rand]
    t = torch.tensor(vals, dtype=torch.float32)
    bf = t.to(torch.bfloat16).view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()
    hf = t.to(torch.float16).view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).tolist()
    (HERE / "convert.json").write_text(json.dumps({
        "source": f"torch {torch.__version__}",
        "f32_bits": [f32_bits(v) for v in vals], "bf16": bf, "f16": hf}, indent=1))

    xs = [-60.0, 60.0, 0.0, -1e-3, 1e-3, -3.0, 3.0, -8.0, 8.0, 15.0, -15.0] + (rng.uniform(-8, 8, 100)).tolist()
    g = torch.nn.functional.gelu(torch.tensor(xs, dtype=torch.float64), approximate="tanh").tolist()
    (HERE / "gelu.json").write_text(json.dumps({"source": f"torch {torch.__version__}", "x": xs, "gelu": g}, indent=1))

    cases = []
    for rows, d, eps, offset, mod in ((3, 16, 1e-5, 1.0, False), (3, 16, 1e-5, 0.0, True), (2, 128, 1e-6, 1.0, True),
                                      (1, 512, 1e-6, 1.0, True), (2, 7, 1e-5, 0.0, False)):
        x = rng.uniform(-3, 3, rows * d).astype(np.float32)
        w = rng.uniform(-0.5, 0.5, d).astype(np.float32)
        sc = rng.uniform(-0.3, 0.3, d).astype(np.float32) if mod else np.zeros(d, np.float32)
        sh = rng.uniform(-0.3, 0.3, d).astype(np.float32) if mod else np.zeros(d, np.float32)
        t = torch.tensor(x.astype(np.float64)).reshape(rows, d)
        weight = (offset + torch.tensor(w.astype(np.float64))) * (1 + torch.tensor(sc.astype(np.float64)))
        out = torch.nn.functional.rms_norm(t, (d,), weight=weight, eps=eps) + torch.tensor(sh.astype(np.float64))
        cases.append({"rows": rows, "d": d, "eps": eps, "offset": offset, "modulated": mod, "x": x.tolist(),
                      "weight": w.tolist(), "scale": sc.tolist(), "shift": sh.tolist(),
                      "out": out.reshape(-1).tolist()})
    (HERE / "rmsnorm.json").write_text(json.dumps({"source": f"torch {torch.__version__}", "cases": cases}))


if __name__ == "__main__":
    main()
