"""An independent Llama implementation to check against: Hugging Face
transformers' LlamaForCausalLM (CPU, fp32, random weights), with its
parameters converted to this repository's llama2.c-convention arrays the way
llama2.c's export.py does for Hugging Face checkpoints: q and k rows permuted
from rotate-half to interleaved RoPE pairs (``permute_reverse``), gate_proj
= w1, up_proj = w3, down_proj = w2.  transformers and torch ship with the
image; nothing here reads the reference.  Used by tests only."""
import numpy as np

import oracle


def hf_model(cfg: oracle.LlamaConfig, seed: int):
    """A random-initialised LlamaForCausalLM of cfg's shape (untied
    classifier, no biases), norm weights drawn around 1."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    hc = LlamaConfig(vocab_size=cfg.vocab, hidden_size=cfg.dim, intermediate_size=cfg.hidden,
                     num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads,
                     num_key_value_heads=cfg.n_kv_heads, max_position_embeddings=cfg.max_seq,
                     rms_norm_eps=cfg.eps, rope_theta=cfg.theta, tie_word_embeddings=False,
                     attention_bias=False, mlp_bias=False, initializer_range=0.05)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(hc).float().eval()
    with torch.no_grad():
        for mod in m.modules():
            if type(mod).__name__ == "LlamaRMSNorm":
                mod.weight.copy_(1.0 + 0.1 * torch.randn_like(mod.weight))
    return m


def _permute_reverse(w, n_heads):
    # rows of each head (h, half, i) -> (h, i, half): the first and second
    # halves of a rotate-half head become the interleaved (2i, 2i + 1) pairs
    d1, d2 = w.shape
    return w.view(n_heads, 2, d1 // n_heads // 2, d2).transpose(1, 2).reshape(d1, d2)


def to_arrays(m, cfg: oracle.LlamaConfig) -> dict:
    """fp32 arrays named and shaped as oracle.weight_shapes."""
    import torch

    sd = {k: v.detach().float() for k, v in m.state_dict().items()}
    per_layer = lambda name: [sd[f"model.layers.{l}.{name}.weight"] for l in range(cfg.n_layers)]
    stack = lambda ts: np.ascontiguousarray(torch.stack(ts).numpy().astype(np.float32))
    return {
        "tok_emb": np.ascontiguousarray(sd["model.embed_tokens.weight"].numpy()),
        "rms_att": stack(per_layer("input_layernorm")),
        "rms_ffn": stack(per_layer("post_attention_layernorm")),
        "wq": stack([_permute_reverse(w, cfg.n_heads) for w in per_layer("self_attn.q_proj")]),
        "wk": stack([_permute_reverse(w, cfg.n_kv_heads) for w in per_layer("self_attn.k_proj")]),
        "wv": stack(per_layer("self_attn.v_proj")),
        "wo": stack(per_layer("self_attn.o_proj")),
        "w1": stack(per_layer("mlp.gate_proj")),
        "w2": stack(per_layer("mlp.down_proj")),
        "w3": stack(per_layer("mlp.up_proj")),
        "rms_final": np.ascontiguousarray(sd["model.norm.weight"].numpy()),
        "wcls": np.ascontiguousarray(sd["lm_head.weight"].numpy()),
    }


def logits(m, tokens) -> np.ndarray:
    """[len(tokens), vocab] logits of one causal forward over the tokens."""
    import torch

    with torch.no_grad():
        return m(torch.tensor([list(tokens)])).logits[0].numpy().astype(np.float64)


def greedy(m, prompt, steps: int):
    """The reference's greedy loop over the forward above: the prompt is
    forced, then each argmax is fed back; returns the tokens after the
    prompt and each step's top-2 logit margin."""
    toks, margins = list(prompt), []
    for _ in range(steps):
        row = logits(m, toks)[-1]
        top2 = np.sort(row)[-2:]
        margins.append(float(top2[1] - top2[0]))
        toks.append(int(np.argmax(row)))
    return toks[len(prompt):], margins
