"""The PyTorch CPU fp32 restatement that bench.py times as its CPU baseline (oracle/torch_cpu.py) computes the same
layers as the fp64 C oracle: gated-delta (chunked form, a partial last chunk, the final state) and GQA (f16-free
path of the oracle), on the synthetic inputs of the benchmark configs at small T. A baseline that computed
something else would time the wrong work."""
import numpy as np
import pytest
import torch

import oracle
import synth
import torch_cpu


@pytest.mark.parametrize("T,B", [(64, 1), (150, 2)])
def test_gdn_layer_matches_oracle(T, B):
    x = synth.gdn_rows(T, B, seed=5)
    p = synth.gdn_params(seed=5)
    y, S = torch_cpu.gdn_layer(torch.from_numpy(x), torch.from_numpy(p["conv"]), torch.from_numpy(p["neg_exp_A"]),
                               torch.from_numpy(p["dt_bias"]), torch.from_numpy(p["gnorm"]))
    for b in range(B):
        st = oracle.GdnState()
        ref = oracle.gdn_forward(x[b], p, st)
        assert oracle.rel_err(y[b].numpy(), ref) < 2e-5
        assert oracle.rel_err(S[b].numpy(), st.S) < 2e-5


def test_gqa_layer_matches_oracle():
    T, B = 100, 2
    x = synth.gqa_rows(T, B, seed=6).astype(np.float32)
    p = synth.gqa_params(seed=6, noise=0.1)
    cos, sin = torch_cpu.rope_table(T)
    y = torch_cpu.gqa_layer(torch.from_numpy(x), torch.from_numpy(p["q_norm"]), torch.from_numpy(p["k_norm"]), cos, sin)
    rope = oracle.rope_table(T, 64, 1e7)
    for b in range(B):
        ref = oracle.gqa_forward(x[b], p, oracle.GqaCache(T), rope, f16=False)
        assert oracle.rel_err(y[b].numpy(), ref) < 1e-5
