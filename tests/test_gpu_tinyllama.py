"""TinyLlama-shape decoder layers on the GPU against the oracle (greedy workload).

The layer shape is TinyLlama-1.1B's (hidden 2048, SwiGLU intermediate 5632, 32
query / 4 KV heads of 64, vocab 32000, RMSNorm eps 1e-5, RoPE theta 10000), W4 g64
weights N(0, 0.02), bf16 embedding.  Two of the 22 layers keep the fp64/fp32
oracle's dequantized weights small; every kernel runs at the real per-layer
sizes.  Greedy decode of 32 tokens from a 32-token prompt of uniform-random ids
(seed 0), checked step by step against the teacher-forced oracle, plus the
prefill logits.
"""
import numpy as np
import pytest
import torch

from oracle.decoder import DecoderShape, OracleDecoder, random_decoder_weights
from shardcompute_amd.executor import ParallelExecutor
from tests.gpu_util import dev
from tests.test_gpu_model import LOGIT_TOL, _margin_check, build_model, logits_np, rel, run

pytestmark = pytest.mark.gpu

SHAPE = DecoderShape(vocab_size=32000, hidden_size=2048, num_layers=2, num_heads=32, num_kv_heads=4,
                     intermediate_size=5632, rope_theta=10000.0)


@pytest.fixture(scope="module")
def weights():
    return random_decoder_weights(SHAPE, seed=0)


@pytest.fixture(scope="module")
def model(weights):
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return build_model(SHAPE, weights, max_pos=512)


def test_tinyllama_shape_prefill_logits(device, weights, model):
    ids = np.random.default_rng(0).integers(0, SHAPE.vocab_size, (1, 32))
    got, _ = run(model.forward(dev(ids.astype(np.int64))))
    ref = OracleDecoder(SHAPE, weights).forward(ids)
    err = rel(logits_np(got), ref)
    print(f"tinyllama-shape prefill logits max-abs-rel {err:.2e}", flush=True)
    assert err <= LOGIT_TOL


def test_tinyllama_shape_greedy_decode(device, weights, model):
    S, n = 32, 32
    ids = np.random.default_rng(0).integers(0, SHAPE.vocab_size, (1, S))
    ex = ParallelExecutor(0, 1, None, model, use_graphs=True)
    out = run(ex.generate(dev(ids.astype(np.int64)), max_new_tokens=n, temperature=0.0)).cpu().numpy()
    assert out.shape == (1, S + n) and np.array_equal(out[:, :S], ids)
    new = out[:, S:]
    _, steps = OracleDecoder(SHAPE, weights).generate_greedy(ids, n, forced=new)
    agree = _margin_check(new, steps)
    print(f"tinyllama-shape greedy: argmax agreement {agree:.2f}", flush=True)
    # every token passed the margin check; exact argmax agreement measured 0.94 (30 of 32;
    # the misses are near-ties of the random-init logits)
    assert agree >= 0.9
