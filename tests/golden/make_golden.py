"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

Each fixture is generated only after the oracle agrees with an independent
float64 numpy restatement of GPT-2 (tests/ref64.py) on the same case, so the
files freeze checked values. Cases:
  tiny_const: rusttorch's unit-test model (gpt2.rs:1023-1082: constant weights)
  tiny_rand : the same tiny config with the seeded synthetic weights
  mini      : V=512, ctx=64, d=128, 2 layers, 2 heads (head_dim 64)
Each stores the prompt, the last-row logits of the prefill plus `decode_steps`
single-token steps, and `n_greedy` greedy ids from generate_cached.

Run: python -m tests.golden.make_golden
"""
import os

import numpy as np

from rusttorch_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = {"tiny_const": (4, 8, 8), "tiny_rand": (4, 8, 8), "mini": (16, 8, 40)}  # prompt, decode steps, greedy


def build_case(name):
    if name == "tiny_const":
        from tests.test_oracle import small_state_dict
        sh = synth.SHAPES["tiny"]
        sd = small_state_dict(sh)
    elif name == "tiny_rand":
        sh = synth.SHAPES["tiny"]
        sd = synth.make_weights(sh)
    else:
        sh = synth.SHAPES["mini"]
        sd = synth.make_weights(sh)
    prompt = synth.make_tokens(CASES[name][0], sh.vocab_size, stream=7)
    return sd, sh, prompt


def main():
    from oracle import oracle as O
    from tests import ref64
    O.build()
    for name, (_, steps, n_greedy) in CASES.items():
        sd, sh, prompt = build_case(name)
        m = O.OracleModel.from_shape(sd, sh)
        c = m.new_cache()
        logits = [m.forward_cached(prompt, c)[-1]]
        toks = list(prompt) + [O.argmax(logits[-1])]
        for _ in range(steps):
            logits.append(m.forward_cached([toks[-1]], c)[0])
            toks.append(O.argmax(logits[-1]))
        ref = ref64.forward(sd, toks[:-1], sh.n_layer, sh.n_head)
        got = np.stack(logits)
        want = ref[len(prompt) - 1:]
        err = np.max(np.abs(got - want))
        assert err < 1e-4, (name, err)
        greedy = m.generate_cached(prompt, n_greedy)
        np.savez(os.path.join(HERE, f"{name}.npz"), prompt=prompt, logits=got, decode_steps=np.int64(steps),
                 n_greedy=np.int64(n_greedy), greedy_ids=np.asarray(greedy, np.uint32))
        print(name, "max |oracle - float64| =", err)


if __name__ == "__main__":
    main()
