"""The linear layers of one decode step, device-resident, replayed as a HIP graph.

A decoder layer of the reference's device runner holds four packed weights,
``w_in`` ([q;k;v] or [q;gate]), ``w_out``, ``w_ffn_gu`` ([gate;up]) and
``w_ffn_dn`` (``metal_cb4_fast_ffi.rs:115-121``, built with
``VxtCb4FastConcatMat::from_subs`` at ``:298-330``), followed by the LM head
(``:143``).  :class:`DecodeStack` runs that projection sequence for one token
(batch 1) with activations in HBM:

    for each layer:  qkv  = W_qkv  . x          (bf16 in, bf16 out)
                     o    = W_o    . qkv[:K_o]   (attention stands in as a slice)
                     gu   = W_gu   . o
                     dn   = W_dn   . gu[:K_dn]   (SwiGLU stands in as a slice)
                     x    = dn
    logits = W_head . x                          (f32 out)

Only the matmuls run (the "matmul-only path"): attention, norms and the
activation function are outside this module, so each projection reads a
slice of the previous one's output instead.  The dependency chain between
launches is the real one.  One token is 4 * layers + 1 launches; captured
once into a HIP graph, it replays with no per-launch host work;
:meth:`DecodeStack.persistent` runs the same token as one persistent launch.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

from . import engine


@dataclass
class LayerWeights:
    """Device tensors of one layer (rows = outputs, cols = inputs)."""

    qkv: engine.GpuPackedTensor
    o: engine.GpuPackedTensor
    gate_up: engine.GpuPackedTensor
    down: engine.GpuPackedTensor


class DecodeStack:
    """One token through ``layers`` decoder layers and the LM head."""

    def __init__(self, eng: engine.HipEngine, layers: Sequence[LayerWeights],
                 lm_head: engine.GpuPackedTensor):
        if not layers:
            raise ValueError("a decode stack needs at least one layer")
        self.eng = eng
        self.layers = list(layers)
        self.lm_head = lm_head
        self.hidden = self.layers[0].qkv.cols
        for i, L in enumerate(self.layers):
            if L.qkv.cols != self.hidden or L.down.rows != self.hidden or L.gate_up.cols != L.o.rows:
                raise ValueError(f"layer {i}: projection shapes do not chain")
            if L.o.cols > L.qkv.rows or L.down.cols > L.gate_up.rows:
                raise ValueError(f"layer {i}: a projection reads past its producer's output")
            if L.o.rows != self.hidden:
                raise ValueError(f"layer {i}: o_proj must map back to the hidden size")
        if lm_head.cols != self.hidden:
            raise ValueError("LM head input size != hidden size")
        big_qkv = max(L.qkv.rows for L in self.layers)
        big_gu = max(L.gate_up.rows for L in self.layers)
        self.x = eng.alloc(self.hidden * 2)            # bf16 token input (never written)
        self.qkv_out = eng.alloc(big_qkv * 2)
        self.o_out = eng.alloc(self.hidden * 2)
        self.gu_out = eng.alloc(big_gu * 2)
        self.dn_out = eng.alloc(self.hidden * 2)
        self.logits = eng.alloc(lm_head.rows * 4)

    # Bytes a token reads from weights (device-resident planes, each once).
    @property
    def weight_bytes(self) -> int:
        ts = [t for L in self.layers for t in (L.qkv, L.o, L.gate_up, L.down)] + [self.lm_head]
        return sum(t.device_bytes for t in ts)

    @property
    def launches(self) -> int:
        return 4 * len(self.layers) + 1

    def set_input(self, x_bf16_bits) -> None:
        """Upload the token's bf16 activations (uint16 bits, [hidden])."""
        self.x.upload(x_bf16_bits)

    def ops(self):
        """The token's projections as ``(tensor, x_ptr, y_ptr, y_dtype)``, in order."""
        bf16, f32 = engine.DTYPE_BF16, engine.DTYPE_F32
        out, x = [], self.x.ptr
        for L in self.layers:
            out += [(L.qkv, x, self.qkv_out.ptr, bf16), (L.o, self.qkv_out.ptr, self.o_out.ptr, bf16),
                    (L.gate_up, self.o_out.ptr, self.gu_out.ptr, bf16),
                    (L.down, self.gu_out.ptr, self.dn_out.ptr, bf16)]
            x = self.dn_out.ptr
        out.append((self.lm_head, x, self.logits.ptr, f32))
        return out

    def persistent(self) -> engine.Chain:
        """The same token as one persistent launch (``HipEngine.chain``): each
        projection's weights stream in while the one before it finishes."""
        return self.eng.chain(self.ops())

    def enqueue(self, stream=None) -> None:
        """Queue one token's projections on ``stream`` (default: the engine's)."""
        stream = stream or self.eng.stream
        for t, xp, yp, ydt in self.ops():
            self.eng.matmul_dev(t, xp, engine.DTYPE_BF16, 1, yp, ydt, stream)

    def capture(self) -> engine.Graph:
        """Record one token into a HIP graph (replay with ``Graph.launch``)."""
        return self.eng.capture(lambda s: self.enqueue(s))

    def free(self) -> None:
        for b in (self.x, self.qkv_out, self.o_out, self.gu_out, self.dn_out, self.logits):
            b.free()
