"""GPU: weights built from safetensors files, and written back.

* Float checkpoints (F32, BF16, F16; several tensors stacked along N, as q/k/v
  into qkv or gate/up into a gated pair) load into exactly the encoding the
  oracle computes from the same f32 rows (bit-exact export).
* Pre-encoded FP8 (per-row and per-tensor scales) and AQ4 tensors load
  bit-exactly.
* save_weights -> load round trips every encoding and layout bit-exactly, and
  the written file reads back through the independent ``safetensors``
  library with the exported tensors.
"""
import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from helpers import activations_bf16, to_torch_bf16, weights

pytestmark = pytest.mark.gpu


def _f32_rows(t):
    return t.float().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("enc", ["fp8", "aq4"])
def test_float_checkpoint_loads_like_the_oracle(uh, orc, gpu, tmp_path, enc, dtype):
    rs = np.random.default_rng(4)
    q = torch.from_numpy((rs.standard_normal((48, 256)) * 0.02).astype(np.float32)).to(dtype)
    k = torch.from_numpy((rs.standard_normal((16, 256)) * 0.02).astype(np.float32)).to(dtype)
    v = torch.from_numpy((rs.standard_normal((16, 256)) * 0.02).astype(np.float32)).to(dtype)
    p = tmp_path / "ckpt.safetensors"
    save_file({"q_proj.weight": q, "k_proj.weight": k, "v_proj.weight": v}, str(p))
    rows = np.concatenate([_f32_rows(q), _f32_rows(k), _f32_rows(v)])
    code = uh.ENCODING_FP8_E4M3_ROW if enc == "fp8" else uh.ENCODING_AQ4_G128
    with uh.SafetensorsFile(p) as f:
        w = uh.load_weight(f, ["q_proj.weight", "k_proj.weight", "v_proj.weight"], code)
    assert (w.n, w.k) == (80, 256)
    ref = orc.fp8_quantize_rows(rows) if enc == "fp8" else orc.aq4_quantize(rows)
    for got, want in zip(w.export(), ref):
        assert np.array_equal(got, want)


def test_gated_pair_from_separate_gate_and_up(uh, orc, gpu, tmp_path):
    rs = np.random.default_rng(5)
    gate = torch.from_numpy((rs.standard_normal((40, 512)) * 0.02).astype(np.float32)).bfloat16()
    up = torch.from_numpy((rs.standard_normal((40, 512)) * 0.02).astype(np.float32)).bfloat16()
    p = tmp_path / "mlp.safetensors"
    save_file({"gate_proj.weight": gate, "up_proj.weight": up}, str(p))
    with uh.SafetensorsFile(p) as f:
        w = uh.load_weight(f, ["gate_proj.weight", "up_proj.weight"],
                           uh.ENCODING_AQ4_G128, gated=True)
    assert w.gated and w.n_out == 40
    rows = np.concatenate([_f32_rows(gate), _f32_rows(up)])
    parts = orc.aq4_quantize(rows)
    for got, want in zip(w.export(), parts):
        assert np.array_equal(got, want)
    xb = activations_bf16(orc, 3, 512, tag=77)
    ref = orc.silu_mul(orc.aq4_gemv(xb, *parts)[0])
    y = w.forward(to_torch_bf16(xb, gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.max(np.abs(y.cpu().numpy() - ref)) <= 1e-2 * np.sqrt(np.mean(ref ** 2))


@pytest.mark.parametrize("scale_shape", ["row", "row1", "tensor"])
def test_encoded_fp8_checkpoint(uh, orc, gpu, tmp_path, scale_shape):
    wf = weights(24, 128, tag=8)
    qc, sc = orc.fp8_quantize_rows(wf)
    if scale_shape == "tensor":
        s_all = np.float32(np.max(sc))
        qc = orc.e4m3_from_f32((orc.e4m3_to_f32(qc) * sc[:, None] / s_all).astype(np.float32))
        s_t, sc = torch.tensor(s_all), np.full(24, s_all, np.float32)
    else:
        s_t = torch.from_numpy(sc) if scale_shape == "row" else torch.from_numpy(sc)[:, None]
    p = tmp_path / "fp8.safetensors"
    save_file({"w": torch.from_numpy(qc).view(torch.float8_e4m3fn), "w_scale": s_t}, str(p))
    with uh.SafetensorsFile(p) as f:
        w = uh.load_weight(f, "w", uh.ENCODING_FP8_E4M3_ROW, scales="w_scale")
    q2, s2 = w.export()
    assert np.array_equal(q2, qc) and np.array_equal(s2, sc)


@pytest.mark.parametrize("enc,gated", [("fp8", False), ("aq4", False), ("aq4", True),
                                       ("fp8", True)])
def test_save_and_load_round_trip(uh, orc, gpu, tmp_path, enc, gated):
    code = uh.ENCODING_FP8_E4M3_ROW if enc == "fp8" else uh.ENCODING_AQ4_G128
    a = uh.LinearWeight.quantize(torch.from_numpy(weights(64, 384, tag=1)).to(gpu), code,
                                 gated=gated)
    b = uh.LinearWeight.quantize(torch.from_numpy(weights(16, 256, tag=2)).to(gpu), code)
    p = tmp_path / "out.safetensors"
    digest = uh.save_weights(p, {"layers.0.mlp": a, "lm_head": b}, {"quantizer": "ullm"})
    with uh.SafetensorsFile(p, sha256=digest) as f:
        assert f.metadata("format") == "ullm-linear"
        assert f.metadata("quantizer") == "ullm"
        assert f.metadata("layers.0.mlp.layout") == ("gated_pairs" if gated else "plain")
        a2 = uh.load_saved_weight(f, "layers.0.mlp")
        b2 = uh.load_saved_weight(f, "lm_head")
    assert a2.gated == gated and a2.n == 64
    for w, w2 in ((a, a2), (b, b2)):
        for x1, x2 in zip(w.export(), w2.export()):
            assert np.array_equal(x1, x2)
    x = torch.randn(5, 384, device=gpu).bfloat16()
    assert torch.equal(a.forward(x), a2.forward(x))
    # the independent reader sees the canonical encodings
    ref = a.export()
    with safe_open(str(p), "np") as g:
        if enc == "fp8":
            assert np.array_equal(g.get_tensor("layers.0.mlp.weight_scale"), ref[1])
            assert g.get_slice("layers.0.mlp.weight").get_dtype() == "F8_E4M3"
        else:
            assert np.array_equal(g.get_tensor("layers.0.mlp.qweight"), ref[0])
            assert np.array_equal(g.get_tensor("layers.0.mlp.scales").view(np.uint16), ref[1])
            assert np.array_equal(g.get_tensor("layers.0.mlp.zeros").view(np.uint16), ref[2])
