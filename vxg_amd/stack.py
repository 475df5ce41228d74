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
once into a HIP graph, it replays with no per-launch host work.
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


@dataclass
class LayerNorms:
    """Device f32 RMSNorm weights of one layer ([hidden] each)."""

    attn: engine.DeviceBuffer
    post_attn: engine.DeviceBuffer


class DecodeStep:
    """One whole decode step for batch 1, token to token on the device.

    The reference CPU step (``forward_step``, llm_cpu.rs:251-482) and the
    device runner (metal_cb4_fast_run.mm:81-92, 355-387) do, per layer::

        normed = rms_norm(cur [+= delta], attn_norm)     vxt_hip_rms_norm_dev
        qkv    = W_qkv . normed                           vxt_hip_matmul_dev
        o      = W_o . attention(qkv)                     (attention stands in
                                                           as the first hidden
                                                           outputs of qkv)
        normed = rms_norm(cur += o, post_attn_norm)       vxt_hip_rms_norm_dev
        act    = act(W_gate . normed) * (W_up . normed)   vxt_hip_ffn_glu_dev
        delta  = W_down . act                             vxt_hip_matmul_dev

    then ``normed = rms_norm(cur += delta, output_norm)``, ``logits =
    W_head . normed``, the greedy id (``vxt_hip_greedy_dev``) and the next
    token's embedding row (``vxt_hip_embed_dev``), which starts the next
    step.  The residual stream ``cur`` and the deltas are f32; the inputs of
    the projections are bf16.  ``embed`` may be the LM head itself (tied
    embeddings, llm_cpu.rs:480).  One step is 6 * layers + 4 launches.

    ``fuse_norm`` (hidden <= 4096): the two RMSNorms of a layer are built
    inside the projections that read them (``vxt_hip_norm_matmul_dev`` for
    [q;k;v] and [gate;up]), the residual stream alternating between two
    buffers (it ends a step in ``cur2``, see ``residual``); bit-identical,
    4 * layers + 4 launches.  The final norm stays a
    launch of its own: every workgroup of the prologue rebuilds the norm, and
    the LM head has thousands of them.
    """

    def __init__(self, eng: engine.HipEngine, layers: Sequence[LayerWeights], norms: Sequence[LayerNorms],
                 output_norm: engine.DeviceBuffer, lm_head: engine.GpuPackedTensor,
                 embed: engine.GpuPackedTensor, eps: float = 1e-6, activation: int = engine.ACT_SILU,
                 embed_scale: float = 1.0, fuse_norm: bool = False):
        if not layers or len(norms) != len(layers):
            raise ValueError("one LayerNorms per layer, at least one layer")
        self.eng, self.layers, self.norms = eng, list(layers), list(norms)
        self.output_norm, self.lm_head, self.embed = output_norm, lm_head, embed
        self.eps, self.activation, self.embed_scale = eps, activation, embed_scale
        self.fuse_norm = fuse_norm
        H = self.hidden = lm_head.cols
        if fuse_norm and H > 4096:
            raise ValueError("the fused norm takes hidden <= 4096")
        if embed.cols != H:
            raise ValueError("embedding width != hidden size")
        for i, L in enumerate(self.layers):
            if L.qkv.cols != H or L.o.rows != H or L.gate_up.cols != H or L.down.rows != H:
                raise ValueError(f"layer {i}: projection shapes do not chain")
            if L.o.cols > L.qkv.rows or L.gate_up.rows % 2 or L.down.cols != L.gate_up.rows // 2:
                raise ValueError(f"layer {i}: o / gate-up / down sizes do not match")
        big_qkv = max(L.qkv.rows for L in self.layers)
        big_ff = max(L.gate_up.rows // 2 for L in self.layers)
        self.cur = eng.alloc(H * 4)
        self.cur2 = eng.alloc(H * 4)       # second residual buffer (fused norms)
        self.delta = eng.alloc(H * 4)
        self.normed = eng.alloc(H * 2)
        self.qkv_out = eng.alloc(big_qkv * 2)
        self.act = eng.alloc(big_ff * 2)
        self.logits = eng.alloc(lm_head.rows * 4)
        self.token = eng.alloc(8)          # [id, nonfinite] from the greedy step

    @property
    def launches(self) -> int:
        return (4 * len(self.layers) + 4) if self.fuse_norm else (6 * len(self.layers) + 4)

    def set_token(self, token: int) -> None:
        import numpy as np
        self.token.upload(np.array([token, 0], np.uint32))

    def read_token(self) -> tuple[int, bool]:
        import numpy as np
        r = self.token.download(np.uint32, (2,))
        return int(r[0]), bool(r[1])

    @property
    def residual(self) -> engine.DeviceBuffer:
        """The buffer holding the residual stream at the end of a step."""
        return self.cur2 if self.fuse_norm else self.cur

    def enqueue(self, stream=None) -> None:
        if self.fuse_norm:
            return self._enqueue_fused(stream)
        e, s = self.eng, stream or self.eng.stream
        bf16, f32 = engine.DTYPE_BF16, engine.DTYPE_F32
        H = self.hidden
        e.embed_dev(self.embed, self.token.ptr, 1, self.cur.ptr, H, self.embed_scale, s)
        for i, (L, N) in enumerate(zip(self.layers, self.norms)):
            e.rms_norm_dev(self.cur.ptr, self.delta.ptr if i else 0, N.attn.ptr, self.normed.ptr, bf16, H, H, 1,
                           self.eps, s)
            e.matmul_dev(L.qkv, self.normed.ptr, bf16, 1, self.qkv_out.ptr, bf16, s)
            e.matmul_dev(L.o, self.qkv_out.ptr, bf16, 1, self.delta.ptr, f32, s)
            e.rms_norm_dev(self.cur.ptr, self.delta.ptr, N.post_attn.ptr, self.normed.ptr, bf16, H, H, 1,
                           self.eps, s)
            e.ffn_glu_dev(L.gate_up, self.normed.ptr, bf16, 1, self.act.ptr, bf16, L.gate_up.rows // 2,
                          self.activation, s)
            e.matmul_dev(L.down, self.act.ptr, bf16, 1, self.delta.ptr, f32, s)
        e.rms_norm_dev(self.cur.ptr, self.delta.ptr, self.output_norm.ptr, self.normed.ptr, bf16, H, H, 1,
                       self.eps, s)
        e.matmul_dev(self.lm_head, self.normed.ptr, bf16, 1, self.logits.ptr, f32, s)
        e.greedy_dev(self.logits.ptr, self.lm_head.rows, self.token.ptr, s)

    def _enqueue_fused(self, stream=None) -> None:
        e, s = self.eng, stream or self.eng.stream
        bf16, f32 = engine.DTYPE_BF16, engine.DTYPE_F32
        H = self.hidden
        bufs, c = (self.cur, self.cur2), 0
        glu = engine.NORM_GLU_GELU_TANH if self.activation == engine.ACT_GELU_TANH else engine.NORM_GLU_SILU
        e.embed_dev(self.embed, self.token.ptr, 1, bufs[0].ptr, H, self.embed_scale, s)

        def normed(t, w, mode, y, ydt, ystride, add):
            nonlocal c
            e.norm_matmul_dev(t, bufs[c].ptr, self.delta.ptr if add else 0, w.ptr, self.eps,
                              bufs[1 - c].ptr if add else 0, mode, y, ydt, ystride, s)
            if add:
                c = 1 - c

        for i, (L, N) in enumerate(zip(self.layers, self.norms)):
            normed(L.qkv, N.attn, engine.NORM_PLAIN, self.qkv_out.ptr, bf16, None, i > 0)
            e.matmul_dev(L.o, self.qkv_out.ptr, bf16, 1, self.delta.ptr, f32, s)
            normed(L.gate_up, N.post_attn, glu, self.act.ptr, bf16, L.gate_up.rows // 2, True)
            e.matmul_dev(L.down, self.act.ptr, bf16, 1, self.delta.ptr, f32, s)
        # 2 * layers - 1 swaps: the stream is in bufs[1] (cur2), where the
        # final add-norm leaves it.
        e.rms_norm_dev(bufs[c].ptr, self.delta.ptr, self.output_norm.ptr, self.normed.ptr, bf16, H, H, 1,
                       self.eps, s)
        e.matmul_dev(self.lm_head, self.normed.ptr, bf16, 1, self.logits.ptr, f32, s)
        e.greedy_dev(self.logits.ptr, self.lm_head.rows, self.token.ptr, s)

    def capture(self) -> engine.Graph:
        """Record one step into a HIP graph; each replay advances one token."""
        return self.eng.capture(lambda s: self.enqueue(s))

    def free(self) -> None:
        for b in (self.cur, self.cur2, self.delta, self.normed, self.qkv_out, self.act, self.logits, self.token):
            b.free()
