"""Writes tests/golden/c2_hf_f32.npz: the Qwen3-1.7B-shaped stack's answer-code probabilities
and final hidden states from HF transformers' Qwen3ForCausalLM, the model
the reference pins its f32 path against (README.md:48, |dp| < 5e-5), on the
seeded weights of that stack at 2 layers and a 4096-token vocab.

Each question is asked alone over [state || question]: the 2048-token state
runs once, and every question continues from a copy of its KV cache with
positions 2048.. (causal attention makes that identical to running the
whole sequence).  The readout is the final-normed hidden state at the
question's last token times the tied head's code rows, softmax in f64.

    python tests/golden/make_c2_hf.py      (CPU only, needs transformers; about a minute)

Not loaded by any test or product code: the tests read the .npz.
"""
import copy
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "rust-cev_amd")]

import numpy as np  # noqa: E402
import torch  # noqa: E402

from cev_hip import configs  # noqa: E402

N_LAYERS, VOCAB, QUESTIONS = 2, 4096, 16


def hf_model(w, W):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=w.vocab, hidden_size=w.hidden, intermediate_size=w.inter, num_hidden_layers=w.n_layers,
                      num_attention_heads=w.hq, num_key_value_heads=w.hkv, head_dim=w.d, hidden_act="silu",
                      max_position_embeddings=8192, rms_norm_eps=w.eps, tie_word_embeddings=True, attention_bias=False,
                      rope_parameters={"rope_type": "default", "rope_theta": w.theta}, use_sliding_window=False)
    cfg._attn_implementation = "eager"
    m = Qwen3ForCausalLM(cfg).to(torch.float32).eval()
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32))  # noqa: E731
    sd = {"model.embed_tokens.weight": t(W["embed"]), "model.norm.weight": t(W["norm"]), "lm_head.weight": t(W["embed"])}
    for i in range(w.n_layers):
        p, q = f"l{i}.", f"model.layers.{i}."
        sd.update({q + "self_attn.q_proj.weight": t(W[p + "wq"]), q + "self_attn.k_proj.weight": t(W[p + "wk"]),
                   q + "self_attn.v_proj.weight": t(W[p + "wv"]), q + "self_attn.o_proj.weight": t(W[p + "wo"]),
                   q + "self_attn.q_norm.weight": t(W[p + "q_norm"]), q + "self_attn.k_norm.weight": t(W[p + "k_norm"]),
                   q + "input_layernorm.weight": t(W[p + "ln1"]), q + "post_attention_layernorm.weight": t(W[p + "ln2"]),
                   q + "mlp.gate_proj.weight": t(W[p + "gate"]), q + "mlp.up_proj.weight": t(W[p + "up"]),
                   q + "mlp.down_proj.weight": t(W[p + "down"])})
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    w = configs.c2(False, n_layers=N_LAYERS, vocab=VOCAB, questions=QUESTIONS)
    t0 = time.time()
    W = w.weights()
    m = hf_model(w, W)
    state, qs, codes = w.ids()
    head = torch.from_numpy(np.ascontiguousarray(W["embed"][codes], np.float32))
    with torch.no_grad():
        out = m.model(input_ids=torch.from_numpy(state[None]), use_cache=True)
        cache = out.past_key_values
        hid, p = [], []
        for q in qs:
            pos = torch.arange(w.state_tokens, w.state_tokens + len(q))[None]
            o = m.model(input_ids=torch.from_numpy(q[None]), past_key_values=copy.deepcopy(cache), position_ids=pos, use_cache=True)
            h = o.last_hidden_state[0, -1].float()
            z = (h @ head.T).double()
            hid.append(h.numpy())
            p.append(torch.softmax(z, dim=-1).numpy())
    p, hid = np.stack(p), np.stack(hid).astype(np.float32)
    print(f"HF Qwen3ForCausalLM, {N_LAYERS} layers, vocab {VOCAB}, {QUESTIONS} questions: {time.time() - t0:.1f} s; p[0] = {np.round(p[0], 5)}")
    np.savez_compressed(os.path.join(HERE, "c2_hf_f32.npz"), p=p, hidden=hid, layers=N_LAYERS, vocab=VOCAB, questions=QUESTIONS)


if __name__ == "__main__":
    main()
