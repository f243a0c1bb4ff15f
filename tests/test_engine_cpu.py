"""Engine harness on the CPU: the Llama decoder against Hugging Face transformers' own
LlamaForCausalLM (random weights written as a local safetensors checkpoint), chunked
prefill, RoPE scaling and the decode-graph buckets. The reference pins its model the same
way, by token identity with HF (tests/test_engine.py:46-94)."""

from __future__ import annotations

import pytest
import torch

from kvserve_amd.engine import ModelConfig
from kvserve_amd.engine.model import build_model, rope_inv_freq
from kvserve_amd.engine.runner import ModelRunner, Sequence, capture_sizes
from tests.engine_backends import TorchRefAttention

transformers = pytest.importorskip("transformers")

TINY = ModelConfig(
    vocab_size=256, hidden_size=64, intermediate_size=160, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
    rms_norm_eps=1e-5, rope_theta=500000.0,
    rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                  "original_max_position_embeddings": 64},
    max_position_embeddings=512, tie_word_embeddings=False,
)  # fmt: skip


@pytest.fixture(scope="module")
def hf_checkpoint(tmp_path_factory):
    torch.manual_seed(0)
    hf_cfg = transformers.LlamaConfig(**{k: v for k, v in TINY.to_hf_dict().items() if k not in ("model_type", "architectures")})
    hf = transformers.LlamaForCausalLM(hf_cfg).float().eval()
    with torch.no_grad():  # less flat than the default init, so argmax is well separated
        for p in hf.parameters():
            if p.dim() == 2:
                p.normal_(0.0, 0.08)
    path = tmp_path_factory.mktemp("tiny_llama")
    hf.save_pretrained(path, safe_serialization=True)
    return hf, path


def _ours(path, max_pos=512):
    return build_model(ModelConfig.from_dir(path), "cpu", torch.float32, max_pos, backend=TorchRefAttention, weights=path)


def test_config_roundtrip(hf_checkpoint):
    _, path = hf_checkpoint
    assert ModelConfig.from_dir(path) == TINY


def test_rope_scaling_matches_transformers():
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    hf_cfg = transformers.LlamaConfig(**{k: v for k, v in TINY.to_hf_dict().items() if k not in ("model_type", "architectures")})
    inv_hf, _ = ROPE_INIT_FUNCTIONS["llama3"](hf_cfg, "cpu")
    torch.testing.assert_close(rope_inv_freq(TINY), inv_hf.float(), rtol=1e-6, atol=0)


def test_logits_match_transformers(hf_checkpoint):
    """All positions of two prompts, through our paged runner (one prefill step each)."""
    hf, path = hf_checkpoint
    ours = _ours(path)
    runner = ModelRunner(ours, num_blocks=64, block_size=16, max_model_len=512, use_graphs=False)
    prompts = [[(7 * i + 3) % 256 for i in range(37)], [(11 * i + 5) % 256 for i in range(19)]]
    seqs = [Sequence(list(p)) for p in prompts]
    # run the prompts as one flat batch and capture the hidden states of every row
    sched = [(s, s.prompt_len) for s in seqs]
    captured = {}
    orig_norm = ours.norm.forward
    ours.norm.forward = lambda x: captured.setdefault("h", orig_norm(x))
    runner.step(sched)
    ours.norm.forward = orig_norm
    logits = ours.compute_logits(captured["h"])
    off = 0
    for p in prompts:
        with torch.no_grad():
            ref = hf(torch.tensor([p])).logits[0].float()
        torch.testing.assert_close(logits[off : off + len(p)], ref, rtol=1e-4, atol=1e-4)
        off += len(p)


def test_greedy_generation_matches_transformers(hf_checkpoint):
    hf, path = hf_checkpoint
    runner = ModelRunner(_ours(path), num_blocks=64, block_size=16, max_model_len=512, use_graphs=False)
    prompts = [[(5 * i + 1) % 256 for i in range(23)], [(3 * i + 2) % 256 for i in range(8)]]
    ours = runner.generate(prompts, max_new_tokens=12)
    for p, got in zip(prompts, ours):
        with torch.no_grad():
            ref = hf.generate(torch.tensor([p]), max_new_tokens=12, do_sample=False, min_new_tokens=12,
                              pad_token_id=0)[0, len(p):].tolist()  # fmt: skip
        assert got == ref


def test_chunked_prefill_gives_the_same_tokens(hf_checkpoint):
    _, path = hf_checkpoint
    prompts = [[(13 * i + 7) % 256 for i in range(41)], [(17 * i + 1) % 256 for i in range(30)], [9]]
    whole = ModelRunner(_ours(path), num_blocks=64, max_model_len=512, use_graphs=False, prefill_token_budget=2048)
    small = ModelRunner(_ours(path), num_blocks=64, max_model_len=512, use_graphs=False, prefill_token_budget=7)
    assert whole.generate(prompts, 6) == small.generate(prompts, 6)


def test_blocks_are_returned_to_the_pool(hf_checkpoint):
    _, path = hf_checkpoint
    r = ModelRunner(_ours(path), num_blocks=16, max_model_len=512, use_graphs=False)
    free = len(r.free_blocks)
    r.generate([[1, 2, 3] * 20], 4)
    assert len(r.free_blocks) == free


def test_capture_sizes_follow_the_reference_buckets():
    assert capture_sizes(1) == [1]
    assert capture_sizes(8) == [1, 2, 4, 8]
    assert capture_sizes(50) == [1, 2, 4, 8, 16, 32, 48, 50]
    assert capture_sizes(128) == [1, 2, 4, 8, 16, 32, 48, 64, 80, 96, 112, 128]
