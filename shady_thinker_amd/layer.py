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
  12-16 tokens on wide linears).
* `prefill` (any number of tokens, f16 activations): the same projections
  through the prefill GEMM, with the down projection on silu(gate) * up
  fused into the GEMM's A pre-pass (`st_gptq_i4_silu_gemm`).

Attention, norms and residuals sit between these calls in a model and are
not part of this path; the caller passes their outputs in.
"""
from __future__ import annotations

from . import model as M
from .weights import GptqWeight

_DECODE_MAX = 32     # tokens per decode call (st_gptq_i4_matvec)
_GATE_UP_BLOCK = 16  # tokens per st_gptq_i4_gate_up_silu call


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
        for w, a, c in ((self.qkv, x, qkv_out), (self.o, attn, o_out), (self.gate, x, gate_out), (self.up, x, up_out)):
            M.gptq_gemm(gpu, a, w.qweight, w.scales, c, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        d = self.down
        M.fused_silu_gptq_gemm(gpu, gate_out, up_out, d.qweight, d.scales, down_out, d.K, d.N, d.group_size,
                               d.qzeros, d.perm, d.flags)
