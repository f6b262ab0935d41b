"""GPU parity of GPT-2 small greedy decoding (
src/models/gpt2_small.sandy.go) against the CPU oracle's op chain
(oracle/gpt2.py): a reduced model step by step (prompt pass and cached
single-token steps, logits at the fp32 tolerance, greedy token wherever the
oracle's top two logits are apart), and the full config-1 run (12 layers,
vocab 50257, 64-token prompt, 32 greedy tokens) against the committed token
sequence of tests/golden/gpt2_c1_greedy.json."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.gpt2 import GPT2Oracle
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gpt2_c1_greedy.json")


@pytest.mark.parametrize("layers,hidden,heads,vocab,prompt_len", [(2, 128, 2, 1000, 8), (3, 256, 4, 3001, 17)])
def test_gpt2_steps_match_oracle(oracle, layers, hidden, heads, vocab, prompt_len):
    from sandyrt_amd.gpt2 import GPT2Config, GPT2Runner, prompt_ids, random_weights
    cfg = GPT2Config(layers=layers, hidden=hidden, heads=heads, head_dim=hidden // heads, ffn=4 * hidden,
                     vocab=vocab, positions=64)
    w = random_weights(cfg, seed=layers)
    prompt = prompt_ids(cfg, prompt_len, seed=layers)
    gpu = GPT2Runner(cfg, w, max_seq=64)
    cpu = GPT2Oracle(oracle, cfg, w)
    ids = list(prompt)
    for step in range(5):
        print(f"gpt2 step {step} ({len(ids)} tokens)", flush=True)
        got = gpu.forward(ids).view(-1).cpu().numpy()
        want = cpu.forward(ids)
        assert_close(got, want, torch.float32, f"logits, step {step}", floor=1.0)  # 12-layer chain
        top2 = np.partition(want, -2)[-2:]
        if top2[1] - top2[0] > 1e-3 * float(np.sqrt(np.mean(want ** 2))):
            assert int(np.argmax(got)) == int(np.argmax(want)), f"greedy token, step {step}"
        ids = [int(np.argmax(want))]
    assert gpu.length == cpu.k[0].shape[2] == prompt_len + 4


def test_gpt2_config1_greedy_tokens_match_cpu():
    """BASELINE config 1 at full size: the GPU's 32 greedy tokens equal the
    CPU reference chain's (the comparison stops at the first step whose CPU
    top-two margin is within the fp32 rounding noise)."""
    from sandyrt_amd.gpt2 import GPT2Config, GPT2Runner, random_weights
    gold = json.load(open(GOLDEN))
    cfg = GPT2Config()
    runner = GPT2Runner(cfg, random_weights(cfg, seed=0), max_seq=128)
    tokens, _, _ = runner.greedy(gold["prompt"], len(gold["tokens"]))
    n = len(tokens)
    for i, m in enumerate(gold["margins"]):
        if m < 1e-4:
            n = i
            break
    assert n >= 8, "the golden run has near-ties too early to compare"
    assert tokens[:n] == gold["tokens"][:n]
