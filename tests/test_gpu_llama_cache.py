"""EntropyDispatchedLlamaBlock with a KV cache (EE/python/dispatch.py:166-209,
214-247) at the reference harness's tiny config (EE/python/benchmark.py:236-246:
hidden 256, FFN 512, 2 layers, 4 Q / 2 KV heads).

The blocks replace the decoder layers of a stock HF LlamaForCausalLM, whose
own forward and generate() then drive them (HF's calling convention:
past_key_values, tensor return).  References: the same HF model with its MLP
weights replaced by the FP16 tier's W8A16 weights (the blocks run the MLP on
that tier without a dispatcher), and the blocks' own forward without a cache."""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _models(attn="eager"):
    pytest.importorskip("transformers")
    from transformers import LlamaConfig, LlamaForCausalLM
    import entropy_engine as ee
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, max_position_embeddings=128, vocab_size=1000,
                      attn_implementation=attn)
    model = LlamaForCausalLM(cfg).cuda().half().eval()
    blocks = [ee.EntropyDispatchedLlamaBlock(l, layer_idx=i).cuda().half().eval()
              for i, l in enumerate(model.model.layers)]
    ref = copy.deepcopy(model)
    with torch.no_grad():
        for l, b in zip(ref.model.layers, blocks):
            l.mlp.gate_proj.weight.copy_(b.gate_proj.weight_f16_nk)
            l.mlp.up_proj.weight.copy_(b.up_proj.weight_f16_nk)
            l.mlp.down_proj.weight.copy_(b.down_proj.weight_f16_nk)
    model.model.layers = torch.nn.ModuleList(blocks)
    return model, ref, blocks


def _close(a, b, tol=2e-2):
    a, b = a.float(), b.float()
    return (a - b).abs().max().item() <= tol * b.abs().max().item()


@pytest.mark.parametrize("attn", ["eager", "sdpa"])
def test_cached_decode_matches_hf_and_uncached(attn):
    from transformers import DynamicCache
    model, ref, blocks = _models(attn)
    g = torch.Generator(device="cuda").manual_seed(1)
    ids = torch.randint(0, 1000, (2, 28), generator=g, device="cuda")
    with torch.no_grad():
        full = model(ids, use_cache=False).logits                 # our blocks, no cache
        full_ref = ref(ids, use_cache=False).logits
        assert _close(full, full_ref)
        c_ours, c_ref = DynamicCache(config=model.config), DynamicCache(config=ref.config)
        o = model(ids[:, :24], past_key_values=c_ours, use_cache=True)
        r = ref(ids[:, :24], past_key_values=c_ref, use_cache=True)
        assert _close(o.logits, r.logits) and _close(o.logits, full[:, :24])
        assert c_ours.get_seq_length() == 24
        for t in range(24, 28):                                   # one token per step
            o = model(ids[:, t:t + 1], past_key_values=c_ours, use_cache=True)
            r = ref(ids[:, t:t + 1], past_key_values=c_ref, use_cache=True)
            assert _close(o.logits[:, -1], r.logits[:, -1]), t
            assert _close(o.logits[:, -1], full[:, t]), t
        assert c_ours.get_seq_length() == 28
        for b in blocks:                                          # each decode step's attention entropy
            assert b.layer_entropy.shape == (2,) and torch.isfinite(b.layer_entropy).all()


def test_generate_with_cache():
    """A few greedy generate() steps through the blocks (use_cache defaults to
    the config's True): every generated token is the argmax of the blocks'
    uncached logits at its position (or within rounding of a tie)."""
    model, _, _ = _models()
    ids = torch.randint(0, 1000, (2, 12), generator=torch.Generator(device="cuda").manual_seed(2), device="cuda")
    with torch.no_grad():
        a = model.generate(ids, max_new_tokens=5, do_sample=False)
        assert a.shape == (2, 17) and torch.equal(a[:, :12], ids)
        full = model(a, use_cache=False).logits.float()
    for t in range(12, 17):
        lg = full[:, t - 1]
        chosen = lg.gather(1, a[:, t:t + 1]).squeeze(1)
        assert (lg.max(dim=1).values - chosen <= 2e-2 * lg.abs().max()).all(), t


def test_reference_calling_convention_returns_present_kv():
    """The reference's call (past_key_value=, use_cache=) returns (hidden,
    present_kv): the updated cache when one is given, else this call's (k, v);
    a second call on that cache sees the first call's keys."""
    from transformers import DynamicCache
    model, _, blocks = _models()
    blk = blocks[0]
    B, S = 2, 16
    x = torch.randn(B, S, 256, device="cuda", dtype=torch.float16)
    with torch.no_grad():
        out = blk(x, use_cache=True)
        assert len(out) == 2 and out[0].shape == (B, S, 256)
        k, v = out[1]
        assert k.shape == (B, 2, S, 64) and v.shape == (B, 2, S, 64)
        cache = DynamicCache(config=model.config)
        h1, present = blk(x, past_key_value=cache, use_cache=True)
        assert present is cache and cache.get_seq_length(0) == S
        assert torch.equal(present.layers[0].keys, k)
        h2 = blk(x[:, :1], past_key_value=cache, use_cache=False)
        assert len(h2) == 1 and cache.get_seq_length(0) == S + 1
        assert torch.equal(out[0], h1)
