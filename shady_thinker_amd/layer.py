"""The linear projections of one decoder layer, for decode and for prefill.

The reference's model is hybrid (src/model.rs:669-969): each layer's
attention side is either self-attention or DeltaNet linear attention (the
loader tells them apart by whether `{layer}.self_attn.q_proj.qweight`
exists, src/weights.rs:247-250), and both kinds share the MLP. Per layer and
per token it runs:

* self-attention: q, k and v of the normed input (`gptq_matvec`,
  src/model.rs:694-714; q is `nh * hd * 2` wide, the query and its output
  gate), o of the gated attention output (:727-729);
* DeltaNet: in_proj_qkv and in_proj_z of the normed input (:749-756), the
  convolution / delta rule / norm in one shader (:758-784), then out_proj
  through `fused_silu_gptq_down` on silu(z) * deltanet_output (:786-791);
* the MLP: gate and up of the post-attention normed input (:803-808) and
  `fused_silu_gptq_down` on them (:809-812).

It prefills a prompt one token at a time (src/inference.rs:93-95).
`DecoderLinears` (self-attention) and `DeltaNetLinears` make the same calls
for a block of tokens:

* `decode` (1-32 tokens, f32 activations): the input projections as one
  concatenated linear (q|k|v, or in_proj_qkv|in_proj_z), the output
  projection (o, or out_proj on silu(z) * o through st_gptq_i4_silu_matvec),
  gate/up fused into h = silu(x.Wg) * (x.Wu), down on h;
  every call one decode entry point (the matvec kernels, or the f16-MFMA
  skinny kernel from 5 tokens on wide linears and from 9 on narrow ones).
* `prefill` (any number of tokens, f16 activations): the same projections
  through the prefill GEMM, with the down projections on silu(a) * b fused
  into the GEMM's A pre-pass (`st_gptq_i4_silu_gemm`).

Attention (self or DeltaNet), norms and residuals sit between these calls in
a model and are not part of this path; the caller passes their outputs in.

`DecoderStack` runs the projections of all layers (of either kind, mixed)
and the lm_head as one token step, eagerly or as one captured HIP graph, with
the caller's ops (norms, attention, residual adds) as capturable hooks
between them.
"""
from __future__ import annotations

from . import model as M
from ._lib import call
from .weights import GptqWeight

_DECODE_MAX = 32     # tokens per decode call (st_gptq_i4_matvec)
_GATE_UP_BLOCK = 32  # tokens per st_gptq_i4_gate_up_silu call
_BF16_BLOCK = 8      # tokens per st_bf16_matvec call


def _mv(gpu, name, x, w: GptqWeight, y) -> None:
    M.gptq_matvec(gpu, name, x, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)


class _Mlp:
    """The MLP shared by both layer kinds: gate, up (one fused call) and
    down, all GptqWeights of one group size."""

    def _init_mlp(self, gate: GptqWeight, up: GptqWeight, down: GptqWeight, hidden: int) -> None:
        if gate.K != hidden or up.K != hidden:
            raise ValueError("gate and up must read the hidden size")
        if gate.N != up.N or down.K != gate.N or down.N != hidden:
            raise ValueError("inconsistent MLP shapes")
        if (gate.perm is None) != (up.perm is None) or (gate.perm is not None and not bool((gate.perm == up.perm).all())):
            raise ValueError("gate and up must share their act-order permutation (one fused call)")
        if gate.flags != up.flags or gate.group_size != up.group_size:
            raise ValueError("gate and up must share their layout flags and group size (one fused call)")
        self.gate, self.up, self.down = gate, up, down
        self.inter = gate.N

    def _mlp_decode(self, gpu, xm, h_out, down_out) -> None:
        g, u = self.gate, self.up
        m = M._rows(xm, self.hidden)
        for r0 in range(0, m, _GATE_UP_BLOCK):
            r1 = min(m, r0 + _GATE_UP_BLOCK)
            M.fused_gate_up_silu(gpu, xm[r0:r1], g.qweight, g.scales, u.qweight, u.scales, h_out[r0:r1], g.K, g.N,
                                 g.group_size, gate_qz=g.qzeros, up_qz=u.qzeros, perm=g.perm, flags=g.flags)
        _mv(gpu, "down_proj", h_out, self.down, down_out)

    def _mlp_prefill(self, gpu, xm, gate_out, up_out, down_out) -> None:
        g, u, d = self.gate, self.up, self.down
        M.gate_up_gemm(gpu, xm, g.qweight, g.scales, u.qweight, u.scales, gate_out, up_out, g.K, g.N, g.group_size,
                       g.qzeros, u.qzeros, g.perm, g.flags)
        M.fused_silu_gptq_gemm(gpu, gate_out, up_out, d.qweight, d.scales, down_out, d.K, d.N, d.group_size,
                               d.qzeros, d.perm, d.flags)

    def nbytes(self) -> int:
        return sum(w.nbytes for w in (self.qkv, self.o, self.gate, self.up, self.down))


class DecoderLinears(_Mlp):
    """A self-attention layer: q, k, v, o, gate, up and down GptqWeights
    (all with the same group size; q, k, v on the same input). q, k and v are
    concatenated along N at construction (GptqWeight.cat: values unchanged),
    so `qkv` is the layer's one input projection. q may be the reference's
    gated width (2 * nh * hd, src/model.rs:696) while o reads nh * hd."""

    kind = "self_attn"

    def __init__(self, q: GptqWeight, k: GptqWeight, v: GptqWeight, o: GptqWeight, gate: GptqWeight,
                 up: GptqWeight, down: GptqWeight):
        if not (q.K == k.K == v.K):
            raise ValueError("q, k and v must read the same hidden size")
        if o.N != q.K:
            raise ValueError("o must write the hidden size")
        self.hidden = q.K
        self._init_mlp(gate, up, down, q.K)
        self.qkv = GptqWeight.cat([q, k, v])
        self.splits = (q.N, k.N, v.N)
        self.o = o
        self.attn_dim = o.K

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

    def decode(self, gpu, x, attn, qkv_out, o_out, h_out, down_out, xm=None) -> None:
        """x [M, hidden] and attn [M, attn_dim] f32, M <= 32. Writes
        qkv_out [M, q+k+v] (q, k, v side by side), o_out [M, hidden],
        h_out [M, inter] = silu(xm.Wg) * (xm.Wu) and down_out [M, hidden] =
        h.Wd, all f32; xm (the MLP's input) defaults to x."""
        m = M._rows(x, self.hidden)
        if m > _DECODE_MAX:
            raise ValueError(f"decode: {m} tokens (at most {_DECODE_MAX}; use prefill)")
        _mv(gpu, "qkv_proj", x, self.qkv, qkv_out)
        _mv(gpu, "o_proj", attn, self.o, o_out)
        self._mlp_decode(gpu, x if xm is None else xm, h_out, down_out)

    def prefill(self, gpu, x, attn, qkv_out, o_out, gate_out, up_out, down_out, xm=None) -> None:
        """x [M, hidden] and attn [M, attn_dim] f16. Writes qkv_out, o_out,
        gate_out [M, inter], up_out [M, inter] and down_out [M, hidden] =
        (silu(gate) * up).Wd, all f16 (each feeds the next GEMM); xm (the
        MLP's input) defaults to x."""
        for w, a, c in ((self.qkv, x, qkv_out), (self.o, attn, o_out)):
            M.gptq_gemm(gpu, a, w.qweight, w.scales, c, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        self._mlp_prefill(gpu, x if xm is None else xm, gate_out, up_out, down_out)


class DeltaNetLinears(_Mlp):
    """A DeltaNet (linear-attention) layer's GPTQ linears
    (LinearAttnWeights, src/weights.rs:24-35): in_proj_qkv [hidden ->
    2 nk kd + nv vd], in_proj_z [hidden -> nv vd], out_proj [nv vd -> hidden],
    and the MLP's gate, up and down. in_proj_qkv and in_proj_z read the same
    normed input and are concatenated along N at construction (`qkv`, outputs
    side by side: the qkv channels, then z); out_proj runs on silu(z) * o, o
    the DeltaNet core's output (src/model.rs:786-791). The layer's other
    weights (conv1d, A_log, dt_bias, norm, the bf16 in_proj_a/b) belong to
    the DeltaNet core, which is the caller's op."""

    kind = "linear_attn"

    def __init__(self, in_qkv: GptqWeight, in_z: GptqWeight, out: GptqWeight, gate: GptqWeight, up: GptqWeight,
                 down: GptqWeight):
        if in_qkv.K != in_z.K:
            raise ValueError("in_proj_qkv and in_proj_z must read the same hidden size")
        if out.K != in_z.N or out.N != in_qkv.K:
            raise ValueError("out_proj must read in_proj_z's width and write the hidden size")
        self.hidden = in_qkv.K
        self._init_mlp(gate, up, down, in_qkv.K)
        self.qkv = GptqWeight.cat([in_qkv, in_z])
        self.splits = (in_qkv.N, in_z.N)
        self.o = out
        self.attn_dim = out.K

    @classmethod
    def from_linears(cls, linears: dict, layer: int, layer_prefix: str = "model.layers") -> "DeltaNetLinears":
        """A DeltaNet layer by the reference loader's names:
        {layer_prefix}.{i}.linear_attn.{in_proj_qkv,in_proj_z,out_proj}
        (src/weights.rs:478-483) and {layer_prefix}.{i}.mlp.{gate,up,down}_proj
        (:494-499)."""
        pfx = f"{layer_prefix}.{layer}"
        names = [f"{pfx}.linear_attn.{p}" for p in ("in_proj_qkv", "in_proj_z", "out_proj")]
        names += [f"{pfx}.mlp.{p}_proj" for p in ("gate", "up", "down")]
        missing = [n for n in names if n not in linears]
        if missing:
            raise KeyError(f"DeltaNetLinears.from_linears: no GPTQ linear {missing[0]}")
        return cls(*(linears[n] for n in names))

    def z_of(self, qkv_out):
        """The z part of the input projection's output [M, qkv.N] (a view;
        contiguous for one token only)."""
        return qkv_out[:, self.splits[0]:]

    def out_proj(self, gpu, z, o, out) -> None:
        """out [M, hidden] = (silu(z) * o) . W_out (fused_silu_gptq_down,
        src/model.rs:786-791); z and o f32 [M, attn_dim]. A z that is not
        contiguous (the z columns of a several-token qkv output) is copied
        out first: the kernels read rows of attn_dim."""
        w = self.o
        if not z.is_contiguous():
            z = z.contiguous()
        M.fused_silu_gptq_down(gpu, z, o, w.qweight, w.scales, out, w.K, w.N, w.group_size, w.qzeros, w.perm,
                               w.flags)

    def decode(self, gpu, x, attn, qkv_out, o_out, h_out, down_out, xm=None) -> None:
        """x [M, hidden] f32 (M <= 32); attn [M, attn_dim] f32 is the DeltaNet
        core's output for this step. Writes qkv_out [M, qkv.N] (the qkv
        channels, then z), o_out [M, hidden] = (silu(z) * attn).W_out, h_out
        and down_out as DecoderLinears.decode; xm defaults to x."""
        m = M._rows(x, self.hidden)
        if m > _DECODE_MAX:
            raise ValueError(f"decode: {m} tokens (at most {_DECODE_MAX}; use prefill)")
        _mv(gpu, "in_proj_qkvz", x, self.qkv, qkv_out)
        self.out_proj(gpu, self.z_of(qkv_out), attn, o_out)
        self._mlp_decode(gpu, x if xm is None else xm, h_out, down_out)

    def prefill(self, gpu, x, attn, qkv_out, o_out, gate_out, up_out, down_out, xm=None) -> None:
        """As decode, with f16 activations and outputs through the prefill
        GEMM (out_proj: st_gptq_i4_silu_gemm on z and attn)."""
        w = self.qkv
        M.gptq_gemm(gpu, x, w.qweight, w.scales, qkv_out, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        z = self.z_of(qkv_out).contiguous()
        d = self.o
        M.fused_silu_gptq_gemm(gpu, z, attn, d.qweight, d.scales, o_out, d.K, d.N, d.group_size, d.qzeros, d.perm,
                               d.flags)
        self._mlp_prefill(gpu, x if xm is None else xm, gate_out, up_out, down_out)


def layer_from_linears(linears: dict, layer: int, layer_prefix: str = "model.layers"):
    """The layer's linears of whichever kind it is: self-attention when
    `{layer_prefix}.{i}.self_attn.q_proj` was loaded (the reference's test,
    src/weights.rs:247-250), DeltaNet otherwise."""
    if f"{layer_prefix}.{layer}.self_attn.q_proj" in linears:
        return DecoderLinears.from_linears(linears, layer, layer_prefix)
    return DeltaNetLinears.from_linears(linears, layer, layer_prefix)


class StackBuffers:
    """Activation buffers of one decode step of a DecoderStack (device
    tensors, f32, `batch` rows): x (normed hidden, input of the input
    projection), qkv (the input projection's outputs side by side), attn (the
    attention side's output: self-attention's gated output, the input of o,
    or the DeltaNet core's output), o (the output projection's), xm (normed
    hidden of the MLP, input of gate/up), h = silu(gate) * up, down, logits;
    and, for DeltaNet layers at several tokens, z (in_proj_z's output, rows
    of its own).

    Layers of different kinds have different widths: qkv and attn are
    per-layer views (`qkv_of(i)`, `attn_of(i)`) of one buffer of the widest
    layer's size, each [batch, width] and contiguous. During a step, `qkv`
    and `attn` are the current layer's views."""

    def __init__(self, gpu, stack: "DecoderStack", batch: int):
        torch = gpu.torch
        L0 = stack.layers[0]
        mk = lambda n: torch.zeros(batch, n, device=gpu.device)
        self.batch = batch
        wq = max(L.qkv.N for L in stack.layers)
        wa = max(L.attn_dim for L in stack.layers)
        self._qkv_flat = torch.zeros(batch * wq, device=gpu.device)
        self._attn_flat = torch.zeros(batch * wa, device=gpu.device)
        self._qkv = [self._qkv_flat[: batch * L.qkv.N].view(batch, L.qkv.N) for L in stack.layers]
        self._attn = [self._attn_flat[: batch * L.attn_dim].view(batch, L.attn_dim) for L in stack.layers]
        dn = [L for L in stack.layers if L.kind == "linear_attn"]
        self.z = mk(max(L.attn_dim for L in dn)) if dn and batch > 1 else None
        self.qkv, self.attn = self._qkv[0], self._attn[0]
        self.x, self.o, self.xm = mk(L0.hidden), mk(L0.hidden), mk(L0.hidden)
        self.h, self.down = mk(L0.inter), mk(L0.hidden)
        self.logits = mk(stack.vocab)

    def qkv_of(self, i: int):
        return self._qkv[i]

    def attn_of(self, i: int):
        return self._attn[i]

    def select(self, i: int) -> None:
        """Make layer i's views the current `qkv` and `attn`."""
        self.qkv, self.attn = self._qkv[i], self._attn[i]


class DecoderStack:
    """The quantized linears of a whole decoder, layer after layer, then the
    lm_head: one token step, run eagerly (`step`) or captured once as a HIP
    graph and replayed per token (`capture`). The reference walks this loop
    on the host and submits once per linear (src/model.rs:348-353, 682-834:
    self-attention q/k/v :694-714 and o :727-729, DeltaNet in_proj_qkv/z
    :749-756 and out_proj :786-791, gate/up/down :803-812, lm_head :824-834).
    Layers are DecoderLinears or DeltaNetLinears, in any mix (the
    reference's hybrid models).

    Between the projections a model runs its own ops (norms, attention or the
    DeltaNet core, residual adds: src/model.rs:685-690, 715-726, 758-784,
    799-802, 820-823). They are outside this path and come in as `hooks`, an
    object with any of these methods, each called with (layer index,
    StackBuffers) and captured into the same graph (so they must be
    capturable stream work, e.g. torch ops on the buffers); when a hook runs,
    b.qkv and b.attn are that layer's views:
      pre_attention(i, b)   fill b.x (layer 0: from the embedding; later:
                            add_rmsnorm of the residual and b.down)
      attention(i, b)       b.qkv -> b.attn (self-attention; for a DeltaNet
                            layer the core's output from its qkv channels)
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
            if (L.hidden, L.inter) != (L0.hidden, L0.inter):
                raise ValueError("DecoderStack: layers of different hidden or intermediate sizes")
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

    @classmethod
    def from_linears(cls, linears: dict, num_layers: int, lm_head, layer_prefix: str = "model.layers"):
        """Every layer of a loaded checkpoint, each of its own kind
        (layer_from_linears), then the lm_head."""
        return cls([layer_from_linears(linears, i, layer_prefix) for i in range(num_layers)], lm_head)

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
            b.select(i)
            if pre:
                pre(i, b)
            _mv(gpu, "qkv_proj", b.x, L.qkv, b.qkv)
            if att:
                att(i, b)
            if L.kind == "self_attn":
                _mv(gpu, "o_proj", b.attn, L.o, b.o)
            else:
                z = L.z_of(b.qkv)
                if m > 1:  # the z columns of several rows: into rows of their own
                    zb = b.z.view(-1)[: m * L.attn_dim].view(m, L.attn_dim)
                    zb.copy_(z)
                    z = zb
                L.out_proj(gpu, z, b.attn, b.o)
            if post:
                post(i, b)
            L._mlp_decode(gpu, b.xm, b.h, b.down)
        if fin:
            fin(b)
        lm = self.lm_head
        if isinstance(lm, GptqWeight):
            _mv(gpu, "lm_head", b.x, lm, b.logits)
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
        return StackGraph(gpu, graph, b)


class StackGraph:
    """A captured DecoderStack step; replay() runs it on torch's current
    stream order (the graph's buffers are the StackBuffers it was captured
    with). Its kernels point into the context's workspace, so the graph pins
    it (st_context_pin_workspace) until release() or garbage collection:
    meanwhile st_context_reserve_workspace refuses to reallocate it. Reserve
    the largest workspace needed before capturing."""

    def __init__(self, gpu, graph, buffers: StackBuffers):
        call("st_context_pin_workspace", gpu.handle, 1)
        self.gpu, self.graph, self.buffers = gpu, graph, buffers

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError("StackGraph: replay after release()")
        self.graph.replay()

    def release(self) -> None:
        """Drop the graph and its workspace pin."""
        if self.graph is not None:
            self.graph = None
            if self.gpu.handle:
                call("st_context_pin_workspace", self.gpu.handle, -1)

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass
