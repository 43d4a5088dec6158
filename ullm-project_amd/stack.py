"""Decode driver for a Llama-3-8B-shaped stack of quantized linear layers.

BASELINE configuration #5: 32 decoder layers (hidden 4096, 32 q / 8 kv heads
x 128, FFN 14336) plus the 128256-row lm_head, every weight AQ4 g128, batch 8
single-token decode.  Only the linear layers are on the path; the reference
defines no attention, norm or activation numerics for it, so two fixed
stand-ins keep the chain well-defined and bounded:

  * attention output = the q slice (first 4096 columns) of the qkv output,
    read in place as a strided view (x_row_stride = 6144);
  * SiLU(gate) * up   = the gate half (first 14336 columns) of the fused
    gate_up output, read in place (x_row_stride = 28672);
  * every projection scales its output by alpha = 1 / (0.02 * sqrt(K)), the
    inverse of the standard deviation a N(0, 0.02^2) weight row gives a unit
    activation, in place of the RMS norms.

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


def layer_shapes(hidden=HIDDEN, qkv=QKV, ffn=FFN):
    """(name, K, N) of the four projections of one decoder layer."""
    return [("qkv", hidden, qkv), ("o", hidden, hidden),
            ("gate_up", hidden, 2 * ffn), ("down", ffn, hidden)]


def aq4_bytes(m, n, k):
    return n * k // 2 + 4 * n * k // 128 + 2 * m * k + 2 * m * n


def step_bytes(m=8, layers=LAYERS, hidden=HIDDEN, qkv=QKV, ffn=FFN, vocab=VOCAB):
    """Algorithmic HBM bytes of one decode step (weights + activations)."""
    per_layer = sum(aq4_bytes(m, n, k) for _, k, n in layer_shapes(hidden, qkv, ffn))
    return layers * per_layer + aq4_bytes(m, vocab, hidden)


class DecodeStack:
    """Owns the AQ4 weights and activation buffers of the stack."""

    def __init__(self, uh, torch, device, batch=8, layers=LAYERS, hidden=HIDDEN,
                 qkv=QKV, ffn=FFN, vocab=VOCAB, seed=0, weights=None):
        self.uh, self.torch, self.dev = uh, torch, device
        self.m, self.layers = batch, layers
        self.hidden, self.qkv, self.ffn, self.vocab = hidden, qkv, ffn, vocab
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
                                                    uh.ENCODING_AQ4_G128)
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
        self.gu_out = torch.empty((batch, 2 * ffn), dtype=bf, device=device)
        self.logits = torch.empty((batch, vocab), dtype=bf, device=device)
        self.alpha_h = 1.0 / (0.02 * math.sqrt(hidden))
        self.alpha_f = 1.0 / (0.02 * math.sqrt(ffn))

    def step(self, stream=None):
        """One decode step: self.h0 -> layers -> self.logits."""
        for i, ws in enumerate(self.weights):
            ws["qkv"].forward(self.h0 if i == 0 else self.h, self.qkv_out,
                              alpha=self.alpha_h, stream=stream)
            ws["o"].forward(self.qkv_out[:, :self.hidden], self.o_out,
                            alpha=self.alpha_h, stream=stream)
            ws["gate_up"].forward(self.o_out, self.gu_out, alpha=self.alpha_h,
                                  stream=stream)
            ws["down"].forward(self.gu_out[:, :self.ffn], self.h,
                               alpha=self.alpha_f, stream=stream)
        self.lm_head.forward(self.h, self.logits, alpha=self.alpha_h, stream=stream)
        return self.logits

    def destroy(self):
        for ws in self.weights:
            for w in ws.values():
                w.destroy()
        self.lm_head.destroy()
