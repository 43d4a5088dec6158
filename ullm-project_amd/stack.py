"""Decode driver for a Llama-3-8B-shaped stack of quantized linear layers.

BASELINE configuration #5: 32 decoder layers (hidden 4096, 32 q / 8 kv heads
x 128, FFN 14336) plus the 128256-row lm_head, every weight AQ4 g128, batch 8
single-token decode.  Only the linear layers are on the path; the reference
defines no attention or norm numerics for it, so fixed stand-ins keep the
chain well-defined and bounded:

  * attention output = the q slice (first 4096 columns) of the qkv output,
    read in place as a strided view (x_row_stride = 6144);
  * MLP activation, by default the pass-through stand-in: the gate half
    (first 14336 columns) of the gate_up output, read in place
    (x_row_stride = 28672).  With swiglu=True it is the real SwiGLU gate
    instead: gate_up is a gated-pair weight (ULLM_LINEAR_LAYOUT_GATED_PAIRS)
    whose forward writes silu(gate) * up [8][14336] directly
    (ULLM_LINEAR_EPILOGUE_SILU_MUL), and down also divides by the RMS of
    silu(g) * u for independent unit normals g, u (0.5965).  SwiGLU is
    quadratic in the scale of its input, so without the RMS norms the
    reference model has between layers a SwiGLU chain drifts away from unit
    RMS (measured x1.08 over the first layer, x3.8 by the fourth, NaN after
    32):
    the 32-layer benchmark keeps the pass-through, the parity test drives
    the SwiGLU chain over a few layers;
  * every projection scales its output by alpha = 1 / (0.02 * sqrt(K)), the
    inverse of the standard deviation a N(0, 0.02^2) weight row gives a unit
    activation, in place of the RMS norms.  (A decoder layer's residual adds
    are available as ULLM_LINEAR_EPILOGUE_RESIDUAL_ADD; without the norms a
    residual stream is not bounded either, so the stand-in chain omits them.)

Per step: 4 x 32 + 1 = 129 forward calls through the C ABI, all on one stream;
the caller may capture them in a HIP graph.
"""
from __future__ import annotations

import math

HIDDEN = 4096
QKV = 6144          # 32 q heads + 2 x 8 kv heads, x 128
FFN = 14336
VOCAB = 128256
LAYERS = 32
# sqrt(E[silu(g)^2]) for g ~ N(0, 1) (numerical quadrature); E[u^2] = 1.
SILU_RMS = 0.5964692


def layer_shapes(hidden=HIDDEN, qkv=QKV, ffn=FFN):
    """(name, K, N) of the four projections of one decoder layer."""
    return [("qkv", hidden, qkv), ("o", hidden, hidden),
            ("gate_up", hidden, 2 * ffn), ("down", ffn, hidden)]


def aq4_bytes(m, n, k, n_out=None):
    return n * k // 2 + 4 * n * k // 128 + 2 * m * k + 2 * m * (n if n_out is None else n_out)


def step_bytes(m=8, layers=LAYERS, hidden=HIDDEN, qkv=QKV, ffn=FFN, vocab=VOCAB,
               swiglu=False):
    """Algorithmic HBM bytes of one decode step (weights + activations; a
    SwiGLU gate_up writes F = n / 2 columns)."""
    per_layer = sum(aq4_bytes(m, n, k, n // 2 if swiglu and name == "gate_up" else None)
                    for name, k, n in layer_shapes(hidden, qkv, ffn))
    return layers * per_layer + aq4_bytes(m, vocab, hidden)


class DecodeStack:
    """Owns the AQ4 weights and activation buffers of the stack."""

    def __init__(self, uh, torch, device, batch=8, layers=LAYERS, hidden=HIDDEN,
                 qkv=QKV, ffn=FFN, vocab=VOCAB, seed=0, weights=None,
                 swiglu=False):
        self.uh, self.torch, self.dev = uh, torch, device
        self.m, self.layers = batch, layers
        self.hidden, self.qkv, self.ffn, self.vocab = hidden, qkv, ffn, vocab
        self.swiglu = swiglu
        shapes = layer_shapes(hidden, qkv, ffn)
        g = torch.Generator(device=device)
        self.weights = []
        for layer in range(layers):
            ws = {}
            for i, (name, k, n) in enumerate(shapes):
                if weights is not None:
                    w = weights[layer][name]
                else:
                    g.manual_seed(seed * 100003 + layer * 16 + i)
                    w = torch.randn((n, k), generator=g, device=device) * 0.02
                ws[name] = uh.LinearWeight.quantize(w.float().contiguous(),
                                                    uh.ENCODING_AQ4_G128,
                                                    gated=swiglu and name == "gate_up")
                del w
            self.weights.append(ws)
        if weights is not None:
            w = weights["lm_head"]
        else:
            g.manual_seed(seed * 100003 + 999)
            w = torch.randn((vocab, hidden), generator=g, device=device) * 0.02
        self.lm_head = uh.LinearWeight.quantize(w.float().contiguous(),
                                                uh.ENCODING_AQ4_G128)
        del w
        bf = torch.bfloat16
        # h0: the step's input token activations (read by layer 0 only, so
        # every step computes the same function of the same input); h: the
        # residual-stream stand-in carried from layer to layer.
        self.h0 = torch.zeros((batch, hidden), dtype=bf, device=device)
        self.h = torch.zeros((batch, hidden), dtype=bf, device=device)
        self.qkv_out = torch.empty((batch, qkv), dtype=bf, device=device)
        self.o_out = torch.empty((batch, hidden), dtype=bf, device=device)
        # MLP activation: silu(gate) * up, or the gate_up output whose gate
        # half down reads in place.
        self.act = torch.empty((batch, ffn if swiglu else 2 * ffn), dtype=bf,
                               device=device)
        self.logits = torch.empty((batch, vocab), dtype=bf, device=device)
        self.alpha_h = 1.0 / (0.02 * math.sqrt(hidden))
        self.alpha_f = 1.0 / (0.02 * math.sqrt(ffn) * (SILU_RMS if swiglu else 1.0))

    def step(self, stream=None):
        """One decode step: self.h0 -> layers -> self.logits."""
        for i, ws in enumerate(self.weights):
            ws["qkv"].forward(self.h0 if i == 0 else self.h, self.qkv_out,
                              alpha=self.alpha_h, stream=stream)
            ws["o"].forward(self.qkv_out[:, :self.hidden], self.o_out,
                            alpha=self.alpha_h, stream=stream)
            ws["gate_up"].forward(self.o_out, self.act, alpha=self.alpha_h,
                                  stream=stream)
            ws["down"].forward(self.act[:, :self.ffn], self.h, alpha=self.alpha_f,
                               stream=stream)
        self.lm_head.forward(self.h, self.logits, alpha=self.alpha_h, stream=stream)
        return self.logits

    def destroy(self):
        for ws in self.weights:
            for w in ws.values():
                w.destroy()
        self.lm_head.destroy()
