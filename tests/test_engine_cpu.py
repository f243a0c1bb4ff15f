"""Engine harness on the CPU: the paged Llama decoder against Hugging Face transformers' own
LlamaForCausalLM (random weights saved as a local safetensors checkpoint and read by the
harness's loader), chunked and mixed steps, RoPE scaling, the pool and the graph buckets. The
reference pins its model the same way, by token identity with HF (tests/test_engine.py:46-94)."""

from __future__ import annotations

import pytest
import torch

from kvserve_amd.attention import build_metadata
from kvserve_amd.engine import ModelConfig
from kvserve_amd.engine.model import apply_rope, build_model, rope_inv_freq, rope_tables
from kvserve_amd.engine.runner import Batcher, ModelRunner, Sequence, decode_buckets, generate, token_buckets
from tests.engine_backends import TorchRefAttention

transformers = pytest.importorskip("transformers")

TINY = ModelConfig(
    vocab_size=256, hidden_size=64, intermediate_size=160, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
    rms_norm_eps=1e-5, rope_theta=500000.0,
    rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                  "original_max_position_embeddings": 64},
    max_position_embeddings=512, tie_word_embeddings=False,
)  # fmt: skip


def _hf_config():
    return transformers.LlamaConfig(**{k: v for k, v in TINY.to_hf_dict().items() if k not in ("model_type", "architectures")})


@pytest.fixture(scope="module")
def hf_checkpoint(tmp_path_factory):
    torch.manual_seed(0)
    hf = transformers.LlamaForCausalLM(_hf_config()).float().eval()
    with torch.no_grad():  # less flat than the default init, so argmax is well separated
        for p in hf.parameters():
            if p.dim() == 2:
                p.normal_(0.0, 0.08)
    path = tmp_path_factory.mktemp("tiny_llama")
    hf.save_pretrained(path, safe_serialization=True)
    return hf, path


def _ours(path, max_pos=512):
    return build_model(ModelConfig.from_dir(path), "cpu", torch.float32, max_pos, backend=TorchRefAttention, weights=path)


def _runner(path, **kw):
    kw.setdefault("num_blocks", 64)
    return ModelRunner(_ours(path), block_size=16, max_model_len=512, **kw)


def test_config_roundtrip(hf_checkpoint):
    _, path = hf_checkpoint
    assert ModelConfig.from_dir(path) == TINY


def test_rope_scaling_matches_transformers():
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    inv_hf, _ = ROPE_INIT_FUNCTIONS["llama3"](_hf_config(), "cpu")
    torch.testing.assert_close(rope_inv_freq(TINY), inv_hf.float(), rtol=1e-6, atol=0)


def test_rope_tables_and_rotation_match_transformers():
    from transformers.models.llama import modeling_llama as hf

    rot = hf.LlamaRotaryEmbedding(_hf_config())
    pos = torch.tensor([[0, 1, 5, 63, 64, 300, 511]])
    x = torch.randn(1, 7, TINY.head_dim)
    cos_hf, sin_hf = rot(x, pos)
    cos, sin = rope_tables(TINY, 512)
    torch.testing.assert_close(cos[pos[0]], cos_hf[0], rtol=0, atol=0)
    torch.testing.assert_close(sin[pos[0]], sin_hf[0], rtol=0, atol=0)
    q = torch.randn(7, TINY.num_heads, TINY.head_dim)
    want, _ = hf.apply_rotary_pos_emb(q.transpose(0, 1)[None], q.transpose(0, 1)[None], cos_hf, sin_hf)
    torch.testing.assert_close(apply_rope(q, cos[pos[0]], sin[pos[0]]), want[0].transpose(0, 1), rtol=0, atol=0)


def test_logits_match_transformers(hf_checkpoint):
    """Every position of two prompts in one flat step through the paged model (two layers of
    write_kv + paged attention), against transformers' forward of each prompt alone."""
    hf, path = hf_checkpoint
    r = _runner(path)
    prompts = [[(7 * i + 3) % 256 for i in range(37)], [(11 * i + 5) % 256 for i in range(19)]]
    seqs = [Sequence(list(p)) for p in prompts]
    for s in seqs:
        s.table = r.pool.take(-(-len(s.tokens) // 16))
    slots = [t * 16 + p % 16 for s in seqs for p, t in ((p, s.table[p // 16]) for p in range(len(s.tokens)))]
    meta = build_metadata("cpu", [s.table for s in seqs], slots, [len(p) for p in prompts], [len(p) for p in prompts],
                          padded_layout=True)  # fmt: skip
    ids = torch.tensor([t for p in prompts for t in p])
    pos = torch.tensor([i for p in prompts for i in range(len(p))])
    logits = r.model.logits(r.model(ids, pos, r.kv_caches, meta))
    off = 0
    for p in prompts:
        with torch.no_grad():
            ref = hf(torch.tensor([p])).logits[0].float()
        torch.testing.assert_close(logits[off : off + len(p)], ref, rtol=1e-4, atol=1e-4)
        off += len(p)


def _hf_greedy(hf, prompt, n):
    with torch.no_grad():
        out = hf.generate(torch.tensor([prompt]), max_new_tokens=n, do_sample=False, min_new_tokens=n, pad_token_id=0)
    return out[0, len(prompt) :].tolist()


def test_greedy_generation_matches_transformers(hf_checkpoint):
    hf, path = hf_checkpoint
    prompts = [[(5 * i + 1) % 256 for i in range(23)], [(3 * i + 2) % 256 for i in range(8)]]
    ours = generate(_runner(path), prompts, max_new_tokens=12)
    for p, got in zip(prompts, ours):
        assert got == _hf_greedy(hf, p, 12)


def test_mixed_steps_with_a_tiny_budget_match_transformers(hf_checkpoint):
    """A 5-token budget and staggered arrivals: prompts are chunked across steps that also carry
    other sequences' decode tokens (the reference's tests/test_engine.py:86-94 budget)."""
    hf, path = hf_checkpoint
    r = _runner(path, token_budget=5)
    b = Batcher(r)
    prompts = [[(13 * i + 7) % 256 for i in range(17)], [(17 * i + 1) % 256 for i in range(9)], [9, 4]]
    seqs = []
    mixed = 0
    for p in prompts:
        seqs.append(b.submit(p, 8))
        b.step()
    while b.busy:
        kinds = {min(s.pending, 2) for s in b.admitted}
        mixed += kinds == {1, 2}
        b.step()
    assert mixed > 0
    for p, s in zip(prompts, seqs):
        assert s.generated == _hf_greedy(hf, p, 8)


def test_chunked_prefill_gives_the_same_tokens(hf_checkpoint):
    _, path = hf_checkpoint
    prompts = [[(13 * i + 7) % 256 for i in range(41)], [(17 * i + 1) % 256 for i in range(30)], [9]]
    whole = generate(_runner(path), prompts, 6, token_budget=2048)
    assert generate(_runner(path), prompts, 6, token_budget=7) == whole


def test_blocks_are_returned_to_the_pool(hf_checkpoint):
    _, path = hf_checkpoint
    r = _runner(path, num_blocks=16)
    free = r.pool.free_blocks
    generate(r, [[1, 2, 3] * 20], 4)
    assert r.pool.free_blocks == free
    with pytest.raises(RuntimeError, match="exhausted"):
        generate(r, [[1] * 300], 2)  # 19 blocks > 16


def test_pool_sized_from_gib(hf_checkpoint):
    """kv_cache_gib -> floor(GiB / (2 L BS Hkv D e)) blocks (reference model_runner.py:94-98)."""
    _, path = hf_checkpoint
    r = ModelRunner(_ours(path), kv_cache_gib=0.001, block_size=16, max_model_len=512)
    per_block = 2 * TINY.num_layers * 16 * TINY.num_kv_heads * TINY.head_dim * 4
    assert r.pool.num_blocks == int(0.001 * 2**30) // per_block
    assert r.kv_caches.shape == (2, 2, r.pool.num_blocks + 1, 16, 2, 16)


def test_max_model_len_is_bounded_by_the_rope_tables(hf_checkpoint):
    """Positions past the model's RoPE tables would be clamped or index out of range: the runner
    refuses a max_model_len above max_positions (the reference builds the model with
    max_positions = max_model_len, model_runner.py:29)."""
    _, path = hf_checkpoint
    with pytest.raises(ValueError, match="RoPE positions"):
        ModelRunner(_ours(path, max_pos=512), num_blocks=8, block_size=16, max_model_len=513)
    assert ModelRunner(_ours(path, max_pos=512), num_blocks=8, block_size=16, max_model_len=512).max_model_len == 512


def test_torch_backend_runs_without_graphs(hf_checkpoint):
    _, path = hf_checkpoint
    r = _runner(path)
    assert r.decode_runner is None and r.piecewise is None and r.dm is None
    generate(r, [[3, 1, 4, 1, 5]], 3)
    assert set(r.paths) == {"eager"}


def test_graph_buckets():
    assert decode_buckets(1) == [1]
    assert decode_buckets(8) == [1, 2, 4, 8]
    assert decode_buckets(50) == [1, 2, 4, 8, 16, 24, 32, 40, 48, 50]
    assert decode_buckets(128) == [1, 2, 4, 8, 16, 24, 32, 40, 48, 56, 64, 96, 128]
    t = token_buckets(2048)
    assert t[:9] == [1, 2, 4, 8, 16, 32, 48, 64, 80] and t[-1] == 2048 and t == sorted(set(t))
    assert token_buckets(24) == [1, 2, 4, 8, 16, 24] and token_buckets(3) == [1, 2, 3]
    # padding past 64 tokens stays within 1/4 of the step
    assert all((b - a) / a <= 0.25 for a, b in zip(t, t[1:]) if a >= 64)
