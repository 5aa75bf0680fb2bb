"""The stacked V-only step on the host (CPU): the oracle's decoder stack
pinned against transformers' Mistral, known answers for the loss and the
norm, and the step's error paths with the reference's texts."""

from __future__ import annotations

import math

import pytest
import torch

from jointkv_amd import v_only
from jointkv_amd.v_only import ClosedLoopRunContext, DecoderStack, v_only_step
from oracle import jointkv_oracle as ref


def stack_dict(stack: DecoderStack) -> dict:
    """A :class:`DecoderStack` as the oracle's plain dict, on the CPU."""

    layers = []
    for w in stack.layers:
        a = w.attention
        layers.append({"input_norm": w.input_norm.cpu(), "post_attention_norm": w.post_attention_norm.cpu(),
                       "q": a.q.cpu(), "k": a.k.cpu(), "v": a.v.cpu(), "o": a.o.cpu(),
                       "gate": w.gate.cpu(), "up": w.up.cpu(), "down": w.down.cpu()})
    return {"embed": stack.embed.cpu(), "final_norm": stack.final_norm.cpu(), "lm_head": stack.lm_head.cpu(),
            "layers": layers}


def _mistral(stack: DecoderStack, vocab: int, hidden: int, inter: int, qh: int, kvh: int):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.MistralConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                                     num_hidden_layers=len(stack.layers), num_attention_heads=qh,
                                     num_key_value_heads=kvh, head_dim=128, sliding_window=4096,
                                     rope_theta=10000.0, rms_norm_eps=1e-5, max_position_embeddings=4096,
                                     tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    model = transformers.MistralForCausalLM(cfg).eval()
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(stack.embed.float())
        model.model.norm.weight.copy_(stack.final_norm.float())
        model.lm_head.weight.copy_(stack.lm_head.float())
        for layer, w in zip(model.model.layers, stack.layers):
            layer.input_layernorm.weight.copy_(w.input_norm.float())
            layer.post_attention_layernorm.weight.copy_(w.post_attention_norm.float())
            for name, t in (("q_proj", w.attention.q), ("k_proj", w.attention.k), ("v_proj", w.attention.v),
                            ("o_proj", w.attention.o)):
                getattr(layer.self_attn, name).weight.copy_(t.float())
            for name, t in (("gate_proj", w.gate), ("up_proj", w.up), ("down_proj", w.down)):
                getattr(layer.mlp, name).weight.copy_(t.float())
    return model


def test_oracle_stack_matches_transformers_mistral():
    # the unadapted oracle stack (raw K/V) against transformers' own Mistral
    # in fp32 with the same weights: pins the block structure (norm
    # placement, residuals, gated MLP, RoPE, GQA, causal mask, lm_head); the
    # oracle rounds every op to fp16 as the device does, hence the tolerance
    vocab, hidden, inter, qh, kvh, tokens = 97, 256, 512, 2, 1, 48
    gen = torch.Generator().manual_seed(4401)
    stack = DecoderStack.synthetic(gen, layers=3, hidden=hidden, kv_heads=kvh, intermediate=inter, vocab=vocab)
    tokens_ids = torch.randint(0, vocab, (1, tokens), generator=gen)
    model = _mistral(stack, vocab, hidden, inter, qh, kvh)
    with torch.no_grad():
        want = model(input_ids=tokens_ids, use_cache=False).logits.float()
        got, codes = ref.stack_logits(tokens_ids, stack_dict(stack), None, None, quantize=False)
    assert codes == [(None, None)] * 3
    scale = float(want.abs().max())
    err = float((got.float() - want).abs().max())
    assert err <= 5e-3 * scale, f"logits max abs error {err} of {scale}"
    # a plausible slip in the block structure is far outside that tolerance
    slipped = stack_dict(stack)
    for w in slipped["layers"]:
        w["input_norm"], w["post_attention_norm"] = w["post_attention_norm"], w["input_norm"]
    with torch.no_grad():
        bad, _ = ref.stack_logits(tokens_ids, slipped, None, None, quantize=False)
    assert float((bad.float() - want).abs().max()) > 10 * err


def test_causal_loss_known_answers():
    # uniform logits: every next token costs log(V)
    tokens = torch.tensor([[3, 1, 4, 1, 5]])
    flat = torch.zeros(1, 5, 7, dtype=torch.float16)
    for fn in (v_only.causal_loss, ref.causal_loss):
        assert float(fn(flat, tokens)) == pytest.approx(math.log(7), rel=1e-6)
    # logit a on the right next token, 0 elsewhere: log(1 + (V-1) e^-a); the
    # last position's logits are never scored
    a = 2.0
    logits = torch.zeros(1, 5, 7)
    for t in range(4):
        logits[0, t, tokens[0, t + 1]] = a
    logits[0, 4] = 100.0
    for fn in (v_only.causal_loss, ref.causal_loss):
        assert float(fn(logits, tokens)) == pytest.approx(math.log(1 + 6 * math.exp(-a)), rel=1e-6)


def test_rms_norm_known_answer():
    # a constant row c has rms |c|: the norm returns weight * sign(c)
    x = torch.tensor([[-3.0, -3.0, -3.0, -3.0], [0.5, 0.5, 0.5, 0.5]], dtype=torch.float16)
    w = torch.tensor([1.0, 2.0, 0.5, -1.0], dtype=torch.float16)
    want = torch.tensor([[-1.0, -2.0, -0.5, 1.0], [1.0, 2.0, 0.5, -1.0]])
    for fn in (v_only.rms_norm, ref.rms_norm):
        got = fn(x, w, 1e-12).float()
        assert torch.allclose(got, want, atol=2e-3)
    # [3, 4]: rms = sqrt(12.5)
    got = v_only.rms_norm(torch.tensor([[3.0, 4.0]]), torch.ones(2), 0.0)
    assert torch.allclose(got, torch.tensor([[3.0, 4.0]]) / math.sqrt(12.5))


def test_synthetic_stack_geometry():
    gen = torch.Generator().manual_seed(1)
    s = DecoderStack.synthetic(gen, layers=2, hidden=512, kv_heads=2, intermediate=64, vocab=11)
    assert len(s.layers) == 2 and s.embed.shape == (11, 512) and s.lm_head.shape == (11, 512)
    a = s.layers[0].attention
    assert (a.query_heads, a.kv_heads) == (4, 2)
    assert s.layers[1].down.shape == (512, 64) and s.layers[1].gate.shape == (64, 512)
    assert all(t.dtype == torch.float16 for t in (s.embed, s.final_norm, a.q, s.layers[0].up))
    for bad in ({"hidden": 500}, {"kv_heads": 3}, {"layers": 0}):
        kw = dict(layers=2, hidden=512, kv_heads=2, intermediate=64, vocab=11) | bad
        with pytest.raises(ValueError, match="geometry"):
            DecoderStack.synthetic(gen, **kw)


class _Codec:
    """Value masters on the CPU; the error paths raise before any HIP call."""

    def __init__(self, *shapes):
        self.key_tables = []
        self.value_tables = torch.nn.ParameterList([torch.nn.Parameter(torch.ones(s)) for s in shapes])


def test_step_rejects_a_nonfinite_loss_and_rate_records():
    ctx = ClosedLoopRunContext(_Codec((2, 3)), "uniform")
    t = ctx.codec.value_tables[0]
    with pytest.raises(RuntimeError, match=r"^nonfinite loss or unexpected rate at step 5$"):
        v_only_step(ctx, lambda: (t.sum() * float("nan"), []), step=4)
    with pytest.raises(RuntimeError, match=r"^nonfinite loss or unexpected rate at step 1$"):
        v_only_step(ctx, lambda: (t.sum() * float("inf"), []), step=0)
    with pytest.raises(RuntimeError, match=r"^nonfinite loss or unexpected rate at step 2$"):
        v_only_step(ctx, lambda: (t.sum(), [{"layer": 0, "request": 0}]), step=1)
    # the check comes before backward: no gradient was written
    assert t.grad is None


def test_step_rejects_missing_and_nonfinite_value_gradients():
    ctx = ClosedLoopRunContext(_Codec((2, 3), (4,)), "uniform")
    first, second = ctx.codec.value_tables
    # the second table takes no gradient
    with pytest.raises(RuntimeError, match=r"^nonfinite/missing V gradient at step 3$"):
        v_only_step(ctx, lambda: (first.sum(), []), step=2)
    # sqrt at 0 has an infinite slope while the loss stays finite
    with torch.no_grad():
        second[1] = 0.0
    with pytest.raises(RuntimeError, match=r"^nonfinite/missing V gradient at step 1$"):
        v_only_step(ctx, lambda: (first.sum() + second.sqrt().sum(), []), step=0)
    assert torch.isinf(second.grad[1])


def test_step_clears_stale_gradients_before_the_loss():
    ctx = ClosedLoopRunContext(_Codec((3,)), "uniform")
    table = ctx.codec.value_tables[0]
    table.grad = torch.full((3,), float("nan"))
    seen = []

    def loss_fn():
        seen.append(table.grad)
        return table.sum() * float("nan"), []

    with pytest.raises(RuntimeError, match="nonfinite loss"):
        v_only_step(ctx, loss_fn, step=0)
    assert seen == [None]


def test_run_context_reset():
    ctx = ClosedLoopRunContext(object(), "uniform")
    ctx.rate_records.append({"layer": 0})
    ctx.reset("dynamic")
    assert ctx.mode == "dynamic" and ctx.rate_records == []


def test_oracle_forced_chain_follows_the_given_codes():
    # forcing the oracle's own codes changes nothing; forcing another first
    # stage makes the chain reconstruct and search from that codeword, while
    # the returned codes stay the oracle's own picks on that chain
    gen = torch.Generator().manual_seed(77)
    states = torch.randn(1, 2, 5, 8, generator=gen).half()
    tables = ref.synthetic_tables(gen, (2, 2, 16, 8), (1.0, 0.5), stage_axis=1)
    out, codes, d1, d2 = ref.hard_residual_vq_exits(states, tables, prefixes=(1, 2), return_margins=True)
    same, codes2, e1, e2 = ref.hard_residual_vq_exits(states, tables, prefixes=(1, 2), return_margins=True,
                                                      forced_codes=codes)
    assert torch.equal(codes2, codes) and torch.equal(e1, d1) and torch.equal(e2, d2)
    assert all(torch.equal(out[k], same[k]) for k in (1, 2))
    forced = codes.clone()
    forced[0, 1, 3, 0] = (int(codes[0, 1, 3, 0]) + 5) % 16
    moved, own, _f1, _f2 = ref.hard_residual_vq_exits(states, tables, prefixes=(1, 2), return_margins=True,
                                                      forced_codes=forced)
    words = tables.half().float()
    first = words[1, 0, int(forced[0, 1, 3, 0])]
    assert torch.equal(moved[1][0, 1, 3], first.half())
    residual = states[0, 1, 3].float() - first
    best = int(((residual[None] - words[1, 1]) ** 2).sum(-1).argmin())
    assert int(own[0, 1, 3, 0]) == int(codes[0, 1, 3, 0]) and int(own[0, 1, 3, 1]) == best
    second = words[1, 1, int(forced[0, 1, 3, 1])]
    assert torch.allclose(moved[2][0, 1, 3].float(), (first + second).half().float())
    # every other row is untouched
    mask = torch.ones(1, 2, 5, dtype=torch.bool)
    mask[0, 1, 3] = False
    assert torch.equal(moved[2][mask], out[2][mask])
