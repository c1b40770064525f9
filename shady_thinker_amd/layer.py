"""The linear projections of one decoder layer, for decode and for prefill.

The reference's `Model::forward` (src/model.rs:669-969) runs, per layer and
per token: q, k and v of the normed input (`gptq_matvec`, :698-714), o of
the attention output (:727-729), gate and up of the post-attention normed
input (:803-808) and `fused_silu_gptq_down` on them (:809-812). It prefills a
prompt one token at a time (src/inference.rs:93-95). `DecoderLinears` makes
the same calls for a block of tokens:

* `decode` (1-32 tokens, f32 activations): q|k|v as one concatenated linear,
  o, gate/up fused into h = silu(x.Wg) * (x.Wu), down on h; every call one
  decode entry point (matvec kernels, or the f16-MFMA skinny kernel for
  9-16 tokens on wide linears).
* `prefill` (any number of tokens, f16 activations): the same projections
  through the prefill GEMM, with the down projection on silu(gate) * up
  fused into the GEMM's A pre-pass (`st_gptq_i4_silu_gemm`).

Attention, norms and residuals sit between these calls in a model and are
not part of this path; the caller passes their outputs in.

`DecoderStack` runs the projections of all layers and the lm_head as one
token step, eagerly or as one captured HIP graph, with the caller's ops
(norms, attention, residual adds) as capturable hooks between them.
"""
from __future__ import annotations

from . import model as M
from .weights import GptqWeight

_DECODE_MAX = 32     # tokens per decode call (st_gptq_i4_matvec)
_GATE_UP_BLOCK = 16  # tokens per st_gptq_i4_gate_up_silu call
_BF16_BLOCK = 8      # tokens per st_bf16_matvec call


class DecoderLinears:
    """q, k, v, o, gate, up and down GptqWeights of one layer (all with the
    same group size; q, k, v on the same input). q, k and v are concatenated
    along N at construction (GptqWeight.cat: values unchanged)."""

    def __init__(self, q: GptqWeight, k: GptqWeight, v: GptqWeight, o: GptqWeight, gate: GptqWeight,
                 up: GptqWeight, down: GptqWeight):
        if not (q.K == k.K == v.K == gate.K == up.K):
            raise ValueError("q, k, v, gate and up must read the same hidden size")
        if gate.N != up.N or down.K != gate.N or o.N != q.K or down.N != q.K:
            raise ValueError("inconsistent layer shapes")
        if (gate.perm is None) != (up.perm is None) or (gate.perm is not None and not bool((gate.perm == up.perm).all())):
            raise ValueError("gate and up must share their act-order permutation (one fused call)")
        if gate.flags != up.flags or gate.group_size != up.group_size:
            raise ValueError("gate and up must share their layout flags and group size (one fused call)")
        self.qkv = GptqWeight.cat([q, k, v])
        self.splits = (q.N, k.N, v.N)
        self.o, self.gate, self.up, self.down = o, gate, up, down
        self.hidden, self.attn_dim, self.inter = q.K, o.K, gate.N

    @classmethod
    def from_linears(cls, linears: dict, layer: int, layer_prefix: str = "model.layers") -> "DecoderLinears":
        """A self-attention layer from load_gptq_checkpoint's {prefix:
        GptqWeight}, by the tensor names the reference's loader takes:
        {layer_prefix}.{i}.self_attn.{q,k,v,o}_proj (src/weights.rs:448-455)
        and {layer_prefix}.{i}.mlp.{gate,up,down}_proj (:494-499)."""
        pfx = f"{layer_prefix}.{layer}"
        names = [f"{pfx}.self_attn.{p}_proj" for p in "qkvo"] + [f"{pfx}.mlp.{p}_proj" for p in ("gate", "up", "down")]
        missing = [n for n in names if n not in linears]
        if missing:
            raise KeyError(f"DecoderLinears.from_linears: no GPTQ linear {missing[0]}")
        return cls(*(linears[n] for n in names))

    def nbytes(self) -> int:
        return sum(w.nbytes for w in (self.qkv, self.o, self.gate, self.up, self.down))

    def decode(self, gpu, x, attn, qkv_out, o_out, h_out, down_out) -> None:
        """x [M, hidden] and attn [M, attn_dim] f32, M <= 32. Writes
        qkv_out [M, q+k+v] (q, k, v side by side), o_out [M, hidden],
        h_out [M, inter] = silu(x.Wg) * (x.Wu) and down_out [M, hidden] =
        h.Wd, all f32."""
        m = M._rows(x, self.hidden)
        if m > _DECODE_MAX:
            raise ValueError(f"decode: {m} tokens (at most {_DECODE_MAX}; use prefill)")
        g = self.gate
        M.gptq_matvec(gpu, "qkv_proj", x, self.qkv.qweight, self.qkv.scales, qkv_out, self.hidden, self.qkv.N,
                      self.qkv.group_size, self.qkv.qzeros, self.qkv.perm, self.qkv.flags)
        M.gptq_matvec(gpu, "o_proj", attn, self.o.qweight, self.o.scales, o_out, self.o.K, self.o.N,
                      self.o.group_size, self.o.qzeros, self.o.perm, self.o.flags)
        for r0 in range(0, m, _GATE_UP_BLOCK):
            r1 = min(m, r0 + _GATE_UP_BLOCK)
            M.fused_gate_up_silu(gpu, x[r0:r1], g.qweight, g.scales, self.up.qweight, self.up.scales, h_out[r0:r1],
                                 self.hidden, self.inter, g.group_size, gate_qz=g.qzeros, up_qz=self.up.qzeros,
                                 perm=g.perm, flags=g.flags)
        d = self.down
        M.gptq_matvec(gpu, "down_proj", h_out, d.qweight, d.scales, down_out, d.K, d.N, d.group_size, d.qzeros,
                      d.perm, d.flags)

    def prefill(self, gpu, x, attn, qkv_out, o_out, gate_out, up_out, down_out) -> None:
        """x [M, hidden] and attn [M, attn_dim] f16. Writes qkv_out, o_out,
        gate_out [M, inter], up_out [M, inter] and down_out [M, hidden] =
        (silu(gate) * up).Wd, all f16 (each feeds the next GEMM)."""
        for w, a, c in ((self.qkv, x, qkv_out), (self.o, attn, o_out)):
            M.gptq_gemm(gpu, a, w.qweight, w.scales, c, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        g, u = self.gate, self.up
        M.gate_up_gemm(gpu, x, g.qweight, g.scales, u.qweight, u.scales, gate_out, up_out, g.K, g.N, g.group_size,
                       g.qzeros, u.qzeros, g.perm, g.flags)
        d = self.down
        M.fused_silu_gptq_gemm(gpu, gate_out, up_out, d.qweight, d.scales, down_out, d.K, d.N, d.group_size,
                               d.qzeros, d.perm, d.flags)


class StackBuffers:
    """Activation buffers of one decode step of a DecoderStack (device
    tensors, f32, `batch` rows): x (normed hidden, input of q|k|v), qkv
    (q, k, v side by side), attn (attention output, input of o), o, xm
    (normed hidden of the MLP, input of gate/up), h = silu(gate) * up,
    down, logits."""

    def __init__(self, gpu, stack: "DecoderStack", batch: int):
        torch = gpu.torch
        L0 = stack.layers[0]
        mk = lambda n: torch.zeros(batch, n, device=gpu.device)
        self.batch = batch
        self.x, self.qkv, self.attn = mk(L0.hidden), mk(L0.qkv.N), mk(L0.attn_dim)
        self.o, self.xm, self.h, self.down = mk(L0.hidden), mk(L0.hidden), mk(L0.inter), mk(L0.hidden)
        self.logits = mk(stack.vocab)


class DecoderStack:
    """The quantized linears of a whole decoder, layer after layer, then the
    lm_head: one token step, run eagerly (`step`) or captured once as a HIP
    graph and replayed per token (`capture`). The reference walks this loop
    on the host and submits once per linear (src/model.rs:348-353, 682-817:
    q/k/v :698-714, o :727-729, gate/up/down :803-812, lm_head :824-834).

    Between the projections a model runs its own ops (norms, attention,
    residual adds: src/model.rs:685-690, 724, 799-802, 820-823). They are
    outside this path and come in as `hooks`, an object with any of these
    methods, each called with (layer index, StackBuffers) and captured into
    the same graph (so they must be capturable stream work, e.g. torch ops
    on the buffers):
      pre_attention(i, b)   fill b.x (layer 0: from the embedding; later:
                            add_rmsnorm of the residual and b.down)
      attention(i, b)       b.qkv -> b.attn
      post_attention(i, b)  b.o (+ residual) -> b.xm
      final(b)              b.down (+ residual) -> b.x, the lm_head's input
    Without hooks the projections run on the buffers as they are (the
    benchmark's synthetic activations); gate/up then reads b.xm and the
    lm_head b.x."""

    def __init__(self, layers: list, lm_head):
        if not layers:
            raise ValueError("DecoderStack: no layers")
        L0 = layers[0]
        for L in layers:
            if (L.hidden, L.attn_dim, L.inter, L.qkv.N) != (L0.hidden, L0.attn_dim, L0.inter, L0.qkv.N):
                raise ValueError("DecoderStack: layers of different shapes")
        self.layers = layers
        self.lm_head = lm_head
        if isinstance(lm_head, GptqWeight):
            if lm_head.K != L0.hidden:
                raise ValueError("DecoderStack: lm_head K differs from the hidden size")
            self.vocab = lm_head.N
        else:  # bf16 [vocab, hidden] (int16 / bfloat16 tensor)
            if lm_head.dim() != 2 or lm_head.shape[1] != L0.hidden:
                raise ValueError("DecoderStack: bf16 lm_head must be [vocab, hidden]")
            self.vocab = lm_head.shape[0]

    def buffers(self, gpu, batch: int) -> StackBuffers:
        if not 1 <= batch <= _DECODE_MAX:
            raise ValueError(f"DecoderStack: batch {batch} (1..{_DECODE_MAX})")
        return StackBuffers(gpu, self, batch)

    def nbytes(self) -> int:
        lm = self.lm_head.nbytes if isinstance(self.lm_head, GptqWeight) else self.lm_head.numel() * 2
        return sum(L.nbytes() for L in self.layers) + lm

    def step(self, gpu, b: StackBuffers, hooks=None) -> None:
        """One token step (all layers, then the lm_head) on b, eagerly."""
        hk = lambda name: getattr(hooks, name, None) if hooks is not None else None
        pre, att, post, fin = hk("pre_attention"), hk("attention"), hk("post_attention"), hk("final")
        m = b.batch
        for i, L in enumerate(self.layers):
            if pre:
                pre(i, b)
            w = L.qkv
            M.gptq_matvec(gpu, "qkv_proj", b.x, w.qweight, w.scales, b.qkv, w.K, w.N, w.group_size, w.qzeros, w.perm,
                          w.flags)
            if att:
                att(i, b)
            w = L.o
            M.gptq_matvec(gpu, "o_proj", b.attn, w.qweight, w.scales, b.o, w.K, w.N, w.group_size, w.qzeros, w.perm,
                          w.flags)
            if post:
                post(i, b)
            g, u = L.gate, L.up
            for r0 in range(0, m, _GATE_UP_BLOCK):
                r1 = min(m, r0 + _GATE_UP_BLOCK)
                M.fused_gate_up_silu(gpu, b.xm[r0:r1], g.qweight, g.scales, u.qweight, u.scales, b.h[r0:r1], g.K, g.N,
                                     g.group_size, gate_qz=g.qzeros, up_qz=u.qzeros, perm=g.perm, flags=g.flags)
            w = L.down
            M.gptq_matvec(gpu, "down_proj", b.h, w.qweight, w.scales, b.down, w.K, w.N, w.group_size, w.qzeros,
                          w.perm, w.flags)
        if fin:
            fin(b)
        lm = self.lm_head
        if isinstance(lm, GptqWeight):
            M.gptq_matvec(gpu, "lm_head", b.x, lm.qweight, lm.scales, b.logits, lm.K, lm.N, lm.group_size, lm.qzeros,
                          lm.perm, lm.flags)
        else:
            for r0 in range(0, m, _BF16_BLOCK):
                r1 = min(m, r0 + _BF16_BLOCK)
                M.bf16_matvec(gpu, b.x[r0:r1], lm, b.logits[r0:r1], lm.shape[1], lm.shape[0])

    def capture(self, gpu, b: StackBuffers, hooks=None) -> "StackGraph":
        """Record one token step as a HIP graph on a side stream (the calls
        are warmed up eagerly first, outside the capture). Replaying it runs
        the whole step on the buffers in b with one launch from the host."""
        torch = gpu.torch
        stream = torch.cuda.Stream(device=gpu.device)
        stream.wait_stream(torch.cuda.current_stream(gpu.device))
        with torch.cuda.stream(stream):
            self.step(gpu, b, hooks)  # warm-up: first-call set-up happens outside the capture
        torch.cuda.current_stream(gpu.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                self.step(gpu, b, hooks)
        torch.cuda.current_stream(gpu.device).wait_stream(stream)
        gpu.sync_stream()
        return StackGraph(graph, b)


class StackGraph:
    """A captured DecoderStack step; replay() runs it on torch's current
    stream order (the graph's buffers are the StackBuffers it was captured
    with)."""

    def __init__(self, graph, buffers: StackBuffers):
        self.graph = graph
        self.buffers = buffers

    def replay(self) -> None:
        self.graph.replay()
