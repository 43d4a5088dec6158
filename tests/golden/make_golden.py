"""Writes the committed fixtures of tests/golden (run from the repo root).

  e4m3_table.npz     all 256 E4M3FN codes and their values, decoded by
                     torch.float8_e4m3fn (a library outside this repo).
  fp8_small.npz      seeded f32 weights [32, 256] and bf16 activations [3, 256],
                     their FP8 row quantization and the fp32-accumulated GEMV.
  aq4_small.npz      the same for AQ4 g128.
  gemm_small.npz     per-token activation quantization and the FP8 GEMM,
                     activations [24, 256], weights [16, 256].
The reference has no implementation of this path (its tree holds no
quantizer, matvec or GEMM), so these vectors come from this build's oracle and
serve as regression vectors for the oracle and the GPU kernels; the oracle
itself is pinned by tests/test_oracle_*.py.
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().parent
SEED = 20260803


def main():
    import torch
    codes = np.arange(256, dtype=np.uint8)
    np.savez_compressed(OUT / "e4m3_table.npz", codes=codes,
             values=torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy())
    rs = np.random.default_rng(SEED)
    w = (rs.standard_normal((32, 256)) * 0.02).astype(np.float32)
    xb = orc.bf16_from_f32(rs.standard_normal((3, 256)).astype(np.float32))
    q, s = orc.fp8_quantize_rows(w)
    np.savez_compressed(OUT / "fp8_small.npz", w=w, x_bf16=xb, q=q, s=s,
             y32=orc.fp8_gemv(xb, q, s)[0])
    p, sc, z = orc.aq4_quantize(w)
    np.savez_compressed(OUT / "aq4_small.npz", w=w, x_bf16=xb, packed=p, scales=sc, zeros=z,
             y32=orc.aq4_gemv(xb, p, sc, z)[0])
    wg = (rs.standard_normal((16, 256)) * 0.02).astype(np.float32)
    xg = orc.bf16_from_f32(rs.standard_normal((24, 256)).astype(np.float32))
    qg, sg = orc.fp8_quantize_rows(wg)
    xq, xs = orc.act_quantize(xg)
    np.savez_compressed(OUT / "gemm_small.npz", w=wg, x_bf16=xg, q=qg, s=sg, xq=xq, xs=xs,
             y32=orc.fp8_gemm(xq, xs, qg, sg)[0])


if __name__ == "__main__":
    main()
