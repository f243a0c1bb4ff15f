"""Engine harness on the GPU: greedy generation through the HIP attention backend is
token-identical to the torch reference backend in fp32 (tests/test_engine.py:85-94 of the
reference), and decode steps replayed from HIP graphs match eager steps
(tests/test_cuda_graph.py:41-82), replay after replay."""

from __future__ import annotations

import pytest
import torch

from kvserve_amd import HipAttention
from kvserve_amd.engine import LLAMA_3_2_1B, ModelConfig
from kvserve_amd.engine.model import build_model
from kvserve_amd.engine.runner import ModelRunner, Sequence
from tests.engine_backends import TorchRefAttention, TorchRefFP8Attention

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(
    vocab_size=2048, hidden_size=512, intermediate_size=1536, num_layers=4, num_heads=8, num_kv_heads=2, head_dim=64,
    rope_scaling=LLAMA_3_2_1B.rope_scaling, tie_word_embeddings=True,
)  # fmt: skip

PROMPTS = [[(31 * i + 7) % 2048 for i in range(n)] for n in (5, 37, 130, 16)]


def _model(backend, dtype, cfg=SMALL, std=0.06):
    return build_model(cfg, "cuda:0", dtype, 1024, backend=backend, seed=1234, std=std)


def test_fp32_greedy_tokens_identical_to_torch_backend(hip_device):
    ref = ModelRunner(_model(TorchRefAttention, torch.float32), num_blocks=128, max_model_len=1024, use_graphs=False)
    want = ref.generate(PROMPTS, max_new_tokens=24)
    hip_eager = ModelRunner(_model(HipAttention, torch.float32), num_blocks=128, max_model_len=1024, use_graphs=False)
    assert hip_eager.generate(PROMPTS, max_new_tokens=24) == want
    hip_graph = ModelRunner(_model(HipAttention, torch.float32), num_blocks=128, max_model_len=1024, use_graphs=True,
                            max_graph_batch=8)  # fmt: skip
    assert hip_graph.generate(PROMPTS, max_new_tokens=24) == want
    assert hip_graph.steps["decode_graph"] == 23


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_replays_match_eager_steps(hip_device, dtype):
    """Two runners with the same weights and prompts: one replays captured decode graphs,
    the other runs eagerly; the logits agree at every one of 6 consecutive steps."""
    runners = [
        ModelRunner(_model(HipAttention, dtype), num_blocks=128, max_model_len=1024, use_graphs=g, max_graph_batch=8)
        for g in (True, False)
    ]
    seqs = [[Sequence(list(p)) for p in PROMPTS[:3]] for _ in runners]
    for r, s in zip(runners, seqs):
        r.prefill(s)
    for step in range(6):
        outs = []
        for r, s in zip(runners, seqs):
            captured = {}
            orig = r.model.compute_logits
            r.model.compute_logits = lambda h, _o=orig, _c=captured: _c.setdefault("l", _o(h))
            r.decode(s)
            r.model.compute_logits = orig
            outs.append(captured["l"])
            torch.cuda.synchronize()
        diff = (outs[0] - outs[1]).abs().max().item()
        scale = outs[1].abs().max().item()
        if dtype == torch.float32:
            assert diff <= 1e-4 * max(1.0, scale), (step, diff, scale)
            assert [x.token_ids for x in seqs[0]] == [x.token_ids for x in seqs[1]]
        else:
            # the graph pads the batch to its bucket, so the bf16 GEMMs may take other kernels
            assert diff <= 3e-2 * scale, (step, diff, scale)
    assert runners[0].steps["decode_graph"] == 6


def test_bf16_llama_1b_shape_runs_and_tracks_the_torch_backend(hip_device):
    """The 1B layer shapes (32 q / 8 kv heads, head_dim 64) in bf16 with two layers: HIP and
    the torch backend agree on the first-step logits within bf16 accuracy, and the greedy
    match rate is reported (bf16 near-ties may flip tokens, as in the reference)."""
    cfg = LLAMA_3_2_1B.with_layers(2)
    prompts = [[(97 * i + 11) % 128000 for i in range(n)] for n in (9, 200, 64)]
    runs = {}
    for name, backend in (("hip", HipAttention), ("torch", TorchRefAttention)):
        r = ModelRunner(_model(backend, torch.bfloat16, cfg, std=0.03), num_blocks=64, max_model_len=1024,
                        use_graphs=backend is HipAttention, max_graph_batch=4)  # fmt: skip
        seqs = [Sequence(list(p)) for p in prompts]
        captured = {}
        orig = r.model.compute_logits
        r.model.compute_logits = lambda h, _o=orig, _c=captured: _c.setdefault("l", _o(h))
        r.prefill(seqs)
        r.model.compute_logits = orig
        for _ in range(15):
            r.decode(seqs)
        runs[name] = (captured["l"], [s.token_ids[len(p):] for s, p in zip(seqs, prompts)])
    l_hip, l_ref = runs["hip"][0], runs["torch"][0]
    assert (l_hip - l_ref).abs().max().item() <= 0.05 * l_ref.abs().max().item()
    match = sum(a == b for x, y in zip(runs["hip"][1], runs["torch"][1]) for a, b in zip(x, y))
    total = sum(len(x) for x in runs["hip"][1])
    print(f"bf16 greedy token match HIP vs torch backend: {match}/{total}")
    assert runs["hip"][1][0][0] == runs["torch"][1][0][0] or match > 0


def test_device_metadata_runner_matches_host_metadata_runner(hip_device):
    """The same fp32 model run with step inputs from kvh_prepare_metadata (resident block
    tables) and from the reference's host path: identical tokens, eager and graph steps, with
    sequences released and their pool rows reused between generations."""
    out = {}
    for dev_meta in (True, False):
        r = ModelRunner(_model(HipAttention, torch.float32), num_blocks=128, max_model_len=1024, use_graphs=True,
                        max_graph_batch=8, device_metadata=dev_meta, prefill_token_budget=64)  # fmt: skip
        assert (r.dm is not None) == dev_meta
        out[dev_meta] = [r.generate(PROMPTS, max_new_tokens=12), r.generate(PROMPTS[::-1], max_new_tokens=12)]
        assert r.steps["decode_graph"] == 22
    assert out[True] == out[False]


def test_fp8_kv_cache_matches_torch_over_the_same_cache_and_graphs_match_eager(hip_device):
    """A bf16 model over an E4M3 KV cache (scales 0.5 / 0.25): the HIP backend's prefill logits
    match the torch backend's over the same E4M3 cache (write: the oracle's quantization;
    attention: fp32 over the dequantized cache) within 5% of the logit scale, as the bf16 test
    above, and decode steps replayed from HIP graphs give the eager steps' logits (3%: the graph
    pads the batch, so the GEMMs may differ)."""

    def with_scales(model):
        for layer in model.layers:
            layer.self_attn.k_scale, layer.self_attn.v_scale = 0.5, 0.25
        return model

    logits = {}
    for name, backend in (("hip", HipAttention), ("torch", TorchRefFP8Attention)):
        r = ModelRunner(with_scales(_model(backend, torch.bfloat16)), num_blocks=128, max_model_len=1024,
                        use_graphs=False, kv_cache_dtype=torch.float8_e4m3fn)  # fmt: skip
        seqs = [Sequence(list(p)) for p in PROMPTS]
        captured = {}
        orig = r.model.compute_logits
        r.model.compute_logits = lambda h, _o=orig, _c=captured: _c.setdefault("l", _o(h))
        r.prefill(seqs)
        logits[name] = captured["l"]
    scale = logits["torch"].abs().max().item()
    assert (logits["hip"] - logits["torch"]).abs().max().item() <= 0.05 * scale
    runners = [
        ModelRunner(with_scales(_model(HipAttention, torch.bfloat16)), num_blocks=128, max_model_len=1024,
                    use_graphs=g, max_graph_batch=8, kv_cache_dtype=torch.float8_e4m3fn)
        for g in (True, False)
    ]  # fmt: skip
    seqs = [[Sequence(list(p)) for p in PROMPTS[:3]] for _ in runners]
    for r, s in zip(runners, seqs):
        r.prefill(s)
    for step in range(4):
        outs = []
        for r, s in zip(runners, seqs):
            captured = {}
            orig = r.model.compute_logits
            r.model.compute_logits = lambda h, _o=orig, _c=captured: _c.setdefault("l", _o(h))
            r.decode(s)
            r.model.compute_logits = orig
            outs.append(captured["l"])
        diff = (outs[0] - outs[1]).abs().max().item()
        assert diff <= 3e-2 * outs[1].abs().max().item(), (step, diff)
    assert runners[0].steps["decode_graph"] == 4
