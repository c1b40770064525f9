"""DecoderStack: a whole decode step (every layer's input projection, output
projection, gate/up, down, then the lm_head) as one captured HIP graph,
against eager execution and against the f64 oracle chained layer by layer,
at configs[4]'s shapes (hidden 2560, 32 query heads of 128 with the
reference's gated q of 2 * 32 * 128 = 8192 columns (src/model.rs:696), k/v
1024, o 4096 -> 2560, intermediate 9728, int4 lm_head 151936), on the
reference's hybrid layer mix: layer 0 self-attention, layer 1 DeltaNet
(in_proj_qkv 2560 -> 6144 and in_proj_z 2560 -> 2048 as one linear, out_proj
2048 -> 2560 on silu(z) * core output; the reference's default head counts,
src/weights.rs:147-151), batch 1 and 16. The reference's loop:
src/model.rs:682-834.

The hooks stand in for the model's norms / attention / DeltaNet core /
residual adds with exact f32 operations (a copy, an add, a multiply by 0.25),
so the numpy restatement of them is bit-exact and the chain's only rounding
is the linears' own (bar: rel-L2 1e-4 of the f64 chain, north_star)."""
import numpy as np
import pytest
import torch

import shady_thinker_amd as sta

pytestmark = pytest.mark.gpu

H, QG, Q, KV, I, V = 2560, 8192, 4096, 1024, 9728, 151936
DT, DZ = 2 * 16 * 128 + 16 * 128, 16 * 128  # DeltaNet qkv channels, z (value heads x value dim)
TOL = 1e-4


class Chain:
    """Layer i > 0 takes layer i-1's down output; self-attention's output =
    its query part / 4, the DeltaNet core's = its first DZ qkv channels / 4;
    the MLP input = (x + o) / 4; the lm_head input = the last down / 4."""

    def __init__(self, kinds):
        self.kinds = kinds

    def pre_attention(self, i, b):
        if i > 0:
            torch.mul(b.down, 0.25, out=b.x)

    def attention(self, i, b):
        n = Q if self.kinds[i] == "self_attn" else DZ
        torch.mul(b.qkv[:, :n], 0.25, out=b.attn)

    def post_attention(self, i, b):
        torch.mul(b.x + b.o, 0.25, out=b.xm)

    def final(self, b):
        torch.mul(b.down, 0.25, out=b.x)


def _weights(gpu, orc, layer, zeros, kind):
    cases, ws = {}, {}
    if kind == "self_attn":
        shapes = (("q", H, QG), ("k", H, KV), ("v", H, KV), ("o", Q, H))
    else:
        shapes = (("in_qkv", H, DT), ("in_z", H, DZ), ("out", DZ, H))
    shapes += (("gate", H, I), ("up", H, I), ("down", I, H))
    for j, (name, k, n) in enumerate(shapes):
        c = orc.gptq_case(500 + 10 * layer + j, k, n, 128, zeros=zeros)
        cases[name] = c
        ws[name] = sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], 128, qzeros=c["qzeros"])
    cls = sta.DecoderLinears if kind == "self_attn" else sta.DeltaNetLinears
    return cases, cls(*(ws[n] for n, _, _ in shapes))


KINDS = ("self_attn", "linear_attn")


@pytest.fixture(scope="module")
def stack(gpu, orc):
    layers, cases = [], []
    for i, kind in enumerate(KINDS):
        c, L = _weights(gpu, orc, i, zeros=(i == 1), kind=kind)
        layers.append(L)
        cases.append(c)
    lmc = orc.gptq_case(599, H, V, 128)
    lm = sta.GptqWeight.upload(gpu, lmc["qweight"], lmc["scales"], 128)
    return sta.DecoderStack(layers, lm), cases, lmc


def _oracle_chain(orc, cases, lmc, x0):
    f32 = np.float32
    lin = lambda c, x, k, n: orc.gptq_matvec_f64(x, c["qweight"], c["scales"], k, n, 128,
                                                 qzeros=c["qzeros"]).astype(f32)
    x = x0.copy()
    down = None
    for i, c in enumerate(cases):
        if i > 0:
            x = down * f32(0.25)
        if KINDS[i] == "self_attn":
            q = lin(c["q"], x, H, QG)
            attn = q[:, :Q] * f32(0.25)
            o = lin(c["o"], attn, Q, H)
        else:
            qkv = lin(c["in_qkv"], x, H, DT)
            z = lin(c["in_z"], x, H, DZ)
            core = qkv[:, :DZ] * f32(0.25)
            hz = orc.silu_gate_f64(z, core)
            o = orc.gptq_matvec_f64(hz, c["out"]["qweight"], c["out"]["scales"], DZ, H, 128,
                                    qzeros=c["out"]["qzeros"]).astype(f32)
        xm = (x + o) * f32(0.25)
        g = orc.gptq_matvec_f64(xm, c["gate"]["qweight"], c["gate"]["scales"], H, I, 128, qzeros=c["gate"]["qzeros"])
        u = orc.gptq_matvec_f64(xm, c["up"]["qweight"], c["up"]["scales"], H, I, 128, qzeros=c["up"]["qzeros"])
        h = orc.silu_gate_f64(g, u).astype(f32)
        down = lin(c["down"], h, I, H)
    x = down * f32(0.25)
    logits = orc.gptq_matvec_f64(x, lmc["qweight"], lmc["scales"], H, V, 128)
    return logits, down


@pytest.mark.parametrize("batch", [1, 16, 32])
def test_stack_replay_equals_eager_and_oracle(gpu, orc, stack, batch):
    st, cases, lmc = stack
    b = st.buffers(gpu, batch)
    x0 = orc.normal_f32(600 + batch, batch * H).reshape(batch, H)
    hooks = Chain(KINDS)

    b.x.copy_(torch.from_numpy(x0))
    st.step(gpu, b, hooks)
    torch.cuda.synchronize()
    eager_logits, eager_down = b.logits.clone(), b.down.clone()

    g = st.capture(gpu, b, hooks)
    other = st.buffers(gpu, batch)
    for rep in range(3):
        b.logits.zero_()
        b.x.copy_(torch.from_numpy(x0))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(b.logits, eager_logits), rep
        assert torch.equal(b.down, eager_down), rep
        other.x.normal_()
        st.step(gpu, other, hooks)  # eager work on the same weights between replays
        torch.cuda.synchronize()

    ref_logits, ref_down = _oracle_chain(orc, cases, lmc, x0)
    e1 = orc.rel_l2(eager_down.cpu().numpy(), ref_down)
    e2 = orc.rel_l2(eager_logits.cpu().numpy(), ref_logits)
    print(f"stack batch {batch}: down rel-L2 {e1:.3e}, logits rel-L2 {e2:.3e}")
    assert e1 < TOL and e2 < TOL


def test_stack_checks(gpu, stack):
    st, _, _ = stack
    with pytest.raises(ValueError):
        st.buffers(gpu, 33)
    with pytest.raises(ValueError):
        sta.DecoderStack([], st.lm_head)
    bad = torch.zeros(V, H + 8, dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError):
        sta.DecoderStack(st.layers, bad)


def test_captured_stack_pins_the_workspace(gpu, stack):
    """A captured step holds pointers into the context workspace: while its
    StackGraph lives, growing the workspace is refused; after release() it
    is allowed again."""
    st, _, _ = stack
    b = st.buffers(gpu, 16)
    g = st.capture(gpu, b)
    big = 1 << 28
    with pytest.raises(sta.ShadyHipError):
        gpu.reserve_workspace(big)
    g.replay()
    torch.cuda.synchronize()
    g.release()
    gpu.reserve_workspace(big)
    with pytest.raises(RuntimeError):
        g.replay()
