"""Engine harness on the GPU.

fp32: greedy generation through the HIP backend is token-identical to the torch reference
backend (the reference's tests/test_engine.py:85-94), including 5-token budgets whose steps mix
prefill chunks with decodes, and the graph paths (decode graphs, piecewise graphs with eager
attention between them) give the eager path's tokens on mixed steps with staggered arrivals
(tests/test_cuda_graph.py:41-58, 112-158 of the reference), with every step on a graph path.
Each of these runs twice: with the backend's fused RoPE + cache write, and with the model
driving the backend exactly as kvserve's Attention.attend does (src/kvserve/model.py:84-108:
torch RoPE, write_kv with v a strided view of the fused QKV output, forward(out=...)).

bf16 (the MFMA, stream-K and merge kernels): teacher-forced against the torch backend, so both
see the same tokens; logits agree within 5% of their scale at every step and at least 90% of
the greedy picks agree (bf16 near-ties may flip, as the reference notes, README.md:306-311).
"""

from __future__ import annotations

from collections import Counter

import pytest
import torch

from kvserve_amd import HipAttention
from kvserve_amd.engine import LLAMA_3_2_1B, ModelConfig
from kvserve_amd.engine.model import build_model
from kvserve_amd.engine.runner import Batcher, ModelRunner, Sequence, generate
from tests.engine_backends import TorchRefAttention, TorchRefFP8Attention

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(
    vocab_size=2048, hidden_size=512, intermediate_size=1536, num_layers=4, num_heads=8, num_kv_heads=2, head_dim=64,
    rope_scaling=LLAMA_3_2_1B.rope_scaling, tie_word_embeddings=True,
)  # fmt: skip

PROMPTS = [[(31 * i + 7) % 2048 for i in range(n)] for n in (5, 37, 130, 16)]


class CountingHip(HipAttention):
    """HipAttention with its entry points counted, and whether write_kv saw a strided v."""

    calls: Counter = Counter()

    @staticmethod
    def write_kv(k_cache, v_cache, k, v, slots, **kw):
        CountingHip.calls["write_kv"] += 1
        CountingHip.calls["strided_v"] += int(not v.is_contiguous())
        return HipAttention.write_kv(k_cache, v_cache, k, v, slots, **kw)

    @staticmethod
    def forward(q, k_cache, v_cache, meta, scale, out=None, **kw):
        CountingHip.calls["forward"] += 1
        CountingHip.calls["forward_out"] += int(out is not None)
        return HipAttention.forward(q, k_cache, v_cache, meta, scale, out=out, **kw)

    @staticmethod
    def rope_and_cache(*a, **kw):
        CountingHip.calls["rope_and_cache"] += 1
        return HipAttention.rope_and_cache(*a, **kw)

    @staticmethod
    def gemv_rope_and_cache(*a, **kw):
        CountingHip.calls["gemv_rope_and_cache"] += 1
        return HipAttention.gemv_rope_and_cache(*a, **kw)


def _hip(fused_rope):
    """The HIP backend for one variant of a test: fused (None) or kvserve's unfused calls
    (False, counted)."""
    CountingHip.calls.clear()
    return HipAttention if fused_rope is None else CountingHip


def _check_unfused_calls(fused_rope) -> None:
    """The unfused variant called write_kv (v strided: a view of the fused QKV output, except
    where a one-token view counts as contiguous) and forward only."""
    if fused_rope is None:
        return
    c = CountingHip.calls
    assert c["write_kv"] > 0 and c["strided_v"] > 0 and c["forward"] > 0, c
    assert c["rope_and_cache"] == 0 and c["gemv_rope_and_cache"] == 0, c


FUSED = pytest.mark.parametrize("fused_rope", [None, False], ids=["fused", "write_kv+forward"])


def _model(backend, dtype, cfg=SMALL, std=0.06, fused_rope=None):
    return build_model(cfg, "cuda:0", dtype, 1024, backend=backend, seed=1234, std=std, fused_rope=fused_rope)


def _runner(backend, dtype, **kw):
    kw.setdefault("num_blocks", 128)
    model = _model(backend, dtype, kw.pop("cfg", SMALL), kw.pop("std", 0.06), kw.pop("fused_rope", None))
    return ModelRunner(model, max_model_len=1024, **kw)


@FUSED
def test_fp32_greedy_tokens_identical_to_torch_backend(hip_device, fused_rope):
    want = generate(_runner(TorchRefAttention, torch.float32), PROMPTS, 24)
    hip = _hip(fused_rope)
    eager = _runner(hip, torch.float32, decode_graphs=False, piecewise_graphs=False, fused_rope=fused_rope)
    assert generate(eager, PROMPTS, 24) == want
    graphs = _runner(hip, torch.float32, max_graph_batch=8, fused_rope=fused_rope)
    assert generate(graphs, PROMPTS, 24) == want
    assert graphs.paths["decode_graph"] == 23 and graphs.paths["piecewise"] == 1, graphs.paths  # 188-token prefill
    _check_unfused_calls(fused_rope)


def _staggered(runner: ModelRunner, prompts, max_new: int, budget: int, forced=None) -> list[list[int]]:
    """New prompts join a running batch one step apart (as tests/test_cuda_graph.py:118-123).
    With `forced`, every sampled token is replaced by forced[prompt][i] (teacher forcing), so
    two backends run the same steps on the same tokens."""
    b = Batcher(runner, budget)
    seqs: list[Sequence] = []

    def step():
        before = [len(s.tokens) for s in seqs]
        b.step()
        if forced is not None:
            for k, (s, n0) in enumerate(zip(seqs, before)):
                if len(s.tokens) > n0:
                    s.tokens[-1] = forced[k][len(s.generated) - 1]

    for p in prompts:
        seqs.append(b.submit(p, max_new))
        step()
    while b.busy:
        step()
    return [s.generated for s in seqs]


def _logits_spy(runner: ModelRunner) -> list[torch.Tensor]:
    """Record the logits of every step the runner samples (ends with the runner)."""
    logs: list[torch.Tensor] = []
    orig = runner.model.logits

    def spy(h):
        out = orig(h)
        logs.append(out)
        return out

    runner.model.logits = spy
    return logs


@FUSED
def test_fp32_five_token_budget_identical_to_torch_backend(hip_device, fused_rope):
    """Every prompt is chunked into 5-token steps that also carry the other sequences' decode
    tokens; HIP with both graph modes gives the torch backend's tokens (the reference's
    tests/test_engine.py:86-93)."""
    prompts = [p[:23] for p in PROMPTS]
    want = _staggered(_runner(TorchRefAttention, torch.float32), prompts, 10, budget=5)
    hip = _runner(_hip(fused_rope), torch.float32, max_graph_batch=8, token_budget=5, fused_rope=fused_rope)
    assert _staggered(hip, prompts, 10, budget=5) == want
    assert hip.paths["piecewise"] > 0 and hip.paths["decode_graph"] > 0 and hip.paths["eager"] == 0, hip.paths
    _check_unfused_calls(fused_rope)
    if fused_rope is not None:  # the piecewise steps' attention wrote into the static buffer
        assert CountingHip.calls["forward_out"] > 0, CountingHip.calls


@FUSED
def test_piecewise_matches_eager_on_mixed_steps(hip_device, fused_rope):
    """A 24-token budget forces chunked prefills mixed with decodes; with graphs every step goes
    through a graph path and the tokens equal eager execution's (the reference's
    tests/test_cuda_graph.py:112-135)."""
    prompts = [p * 3 for p in PROMPTS[:3]] + [PROMPTS[3]]
    hip = _hip(fused_rope)
    eager = _runner(hip, torch.float32, decode_graphs=False, piecewise_graphs=False, token_budget=24,
                    fused_rope=fused_rope)  # fmt: skip
    want = _staggered(eager, prompts, 12, budget=24)
    assert set(eager.paths) == {"eager"}
    g = _runner(hip, torch.float32, max_graph_batch=8, token_budget=24, fused_rope=fused_rope)
    assert g.piecewise.max_tokens == 24  # capped by the step budget
    assert _staggered(g, prompts, 12, budget=24) == want
    assert g.paths["piecewise"] > 0 and g.paths["decode_graph"] > 0 and g.paths["eager"] == 0, g.paths
    _check_unfused_calls(fused_rope)


def test_large_steps_bypass_piecewise(hip_device):
    r = _runner(HipAttention, torch.float32, max_graph_batch=4, token_budget=256, max_piecewise_tokens=64)
    assert r.piecewise.max_tokens == 64
    out = generate(r, [[1000 + i for i in range(200)]], 3)
    assert r.paths["eager"] == 1 and r.paths["decode_graph"] == 2, r.paths
    assert out == generate(_runner(TorchRefAttention, torch.float32), [[1000 + i for i in range(200)]], 3)


def test_piecewise_hidden_states_match_eager(hip_device):
    """One mixed step (a prompt chunk beside three decodes) through the piecewise runner and
    through the eager model: final hidden states within 1e-4 (fp32)."""
    r = _runner(HipAttention, torch.float32, max_graph_batch=4, token_budget=64, device_metadata=False)
    seqs = [Sequence(list(p)) for p in PROMPTS]
    r.prefill(seqs[:3])
    plan = [(s, 1) for s in seqs[:3]] + [(seqs[3], 9)]
    hidden = {}
    orig = r.model.logits
    for path in ("piecewise", "eager"):
        keep = [(s.computed, list(s.tokens)) for s in seqs]
        count = r.paths[path]

        def spy(h, _path=path):
            hidden[_path] = h.clone()
            return orig(h)

        r.model.logits = spy
        r.execute(plan, eager=path == "eager")
        r.model.logits = orig
        assert r.paths[path] == count + 1
        for s, (c, t) in zip(seqs, keep):  # undo the step: the same cache rows are written again
            s.computed, s.tokens = c, t
    torch.testing.assert_close(hidden["piecewise"], hidden["eager"], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_graph_replays_match_eager_steps(hip_device, dtype):
    """Two runners with the same weights and prompts, one replaying decode graphs and one
    eager, the graph runner teacher-forced to the eager runner's tokens: logits agree at each of
    6 consecutive steps (fp32: 1e-4 and the same tokens unforced; bf16: within 3% of the scale,
    as the graph pads the batch to its bucket, so the small-batch GEMMs may pick other kernels)."""
    runners = [_runner(HipAttention, dtype, max_graph_batch=8, decode_graphs=g, piecewise_graphs=False)
               for g in (True, False)]  # fmt: skip
    seqs = [[Sequence(list(p)) for p in PROMPTS[:3]] for _ in runners]
    for r, s in zip(runners, seqs):
        r.prefill(s)
    for step in range(6):
        outs = []
        for r, s in zip(runners, seqs):
            got = {}
            orig = r.model.logits
            r.model.logits = lambda h, _o=orig, _g=got: _g.setdefault("l", _o(h))
            r.decode(s)
            r.model.logits = orig
            outs.append(got["l"])
        if dtype != torch.float32:
            for g, e in zip(seqs[0], seqs[1]):
                g.tokens[-1] = e.tokens[-1]
        diff = (outs[0] - outs[1]).abs().max().item()
        scale = outs[1].abs().max().item()
        if dtype == torch.float32:
            assert diff <= 1e-4 * max(1.0, scale), (step, diff, scale)
            assert [x.tokens for x in seqs[0]] == [x.tokens for x in seqs[1]]
        else:
            assert diff <= 3e-2 * scale, (step, diff, scale)
    assert runners[0].paths["decode_graph"] == 6


def test_graph_padding_never_touches_allocated_blocks(hip_device):
    """A decode step of 3 sequences replayed from the 4-row graph (one padding row): every
    pool byte outside the scratch block and the 3 new tokens' slots is unchanged, in every
    layer (the reference's padding check, tests/test_cuda_graph.py:86-95)."""
    r = _runner(HipAttention, torch.float32, max_graph_batch=4, piecewise_graphs=False, num_blocks=64)
    seqs = [Sequence(list(p)) for p in PROMPTS[:3]]
    r.prefill(seqs)
    before = r.kv_caches.clone()
    bs = r.block_size
    pos = [s.computed for s in seqs]  # the position each sequence's step writes
    r.decode(seqs)
    new = [(s.table[q // bs], q % bs) for s, q in zip(seqs, pos)]
    assert r.paths["decode_graph"] == 1, r.paths
    after = r.kv_caches
    keep = torch.ones(after.shape[2:4], dtype=torch.bool)  # [blocks + 1, BS]
    keep[r.pool.scratch_block] = False
    for blk, off in new:
        keep[blk, off] = False
    keep = keep.to(after.device)
    assert torch.equal(after[:, :, keep], before[:, :, keep])
    for blk, off in new:  # the new rows were written (in every layer)
        assert not torch.equal(after[:, :, blk, off], before[:, :, blk, off])


def test_batched_generation_equals_one_sequence_at_a_time(hip_device):
    """fp32 greedy tokens of four prompts generated together (mixed prefill / decode steps,
    both graph modes) equal those of each prompt generated alone (the reference's batched vs
    single check, tests/test_engine.py:46-94)."""
    together = generate(_runner(HipAttention, torch.float32, max_graph_batch=8, token_budget=64), PROMPTS, 12)
    alone = [generate(_runner(HipAttention, torch.float32, max_graph_batch=8, token_budget=64), [p], 12)[0]
             for p in PROMPTS]  # fmt: skip
    assert together == alone


@FUSED
def test_bf16_llama_1b_shape_tracks_the_torch_backend(hip_device, fused_rope):
    """The Llama-3.2-1B layer shapes (32 q / 8 kv heads, D 64) in bf16 with two layers, a
    48-token budget so prompts are chunked into mixed steps, graphs on: teacher-forced against
    the torch backend, logits within 5% of their scale at every step, >= 90% greedy agreement."""
    cfg = LLAMA_3_2_1B.with_layers(2)
    prompts = [[(97 * i + 11) % 128000 for i in range(n)] for n in (9, 200, 64, 31)]
    ref = _runner(TorchRefAttention, torch.bfloat16, cfg=cfg, std=0.03, num_blocks=64)
    l_ref = _logits_spy(ref)
    forced = _staggered(ref, prompts, 12, budget=48)
    hip = _runner(_hip(fused_rope), torch.bfloat16, cfg=cfg, std=0.03, num_blocks=64, max_graph_batch=4,
                  token_budget=48, fused_rope=fused_rope)  # fmt: skip
    l_hip = _logits_spy(hip)
    assert _staggered(hip, prompts, 12, budget=48, forced=forced) == forced
    assert len(l_ref) == len(l_hip) and hip.paths["piecewise"] > 0 and hip.paths["decode_graph"] > 0, hip.paths
    agree = total = 0
    for step, (a, b) in enumerate(zip(l_hip, l_ref)):
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 0.05 * scale, step
        agree += int((a.argmax(-1) == b.argmax(-1)).sum())
        total += a.shape[0]
    print(f"bf16 greedy agreement HIP vs torch backend (teacher-forced): {agree}/{total}")
    assert agree >= 0.9 * total, (agree, total)
    _check_unfused_calls(fused_rope)


def test_device_metadata_runner_matches_host_metadata_runner(hip_device):
    """The same fp32 model with step inputs from kvh_prepare_metadata (resident block tables)
    and from the reference's host path: identical tokens on every path (decode graph,
    piecewise, eager), with sequences released and pool rows reused between generations."""
    out = {}
    for dev_meta in (True, False):
        r = _runner(HipAttention, torch.float32, max_graph_batch=8, device_metadata=dev_meta, token_budget=64,
                    max_piecewise_tokens=32)  # fmt: skip
        assert (r.dm is not None) == dev_meta
        out[dev_meta] = [_staggered(r, PROMPTS, 12, budget=64), _staggered(r, PROMPTS[::-1], 12, budget=64)]
        assert r.paths["decode_graph"] > 0 and r.paths["piecewise"] > 0 and r.paths["eager"] > 0, r.paths
    assert out[True] == out[False]


def test_fp8_kv_cache_matches_torch_over_the_same_cache_and_graphs_match_eager(hip_device):
    """A bf16 model over an E4M3 KV cache (scales 0.5 / 0.25): the HIP backend's prefill logits
    match the torch backend's over the same E4M3 cache (write: the oracle's quantization;
    attention: fp32 over the dequantized cache) within 5% of the logit scale, and decode steps
    replayed from HIP graphs give the eager steps' logits within 3%."""

    def fp8_runner(backend, **kw):
        model = _model(backend, torch.bfloat16)
        for lw in model.w.layers:  # before the runner: graphs capture the scales as arguments
            lw.k_scale, lw.v_scale = 0.5, 0.25
        return ModelRunner(model, num_blocks=128, max_model_len=1024, kv_cache_dtype=torch.float8_e4m3fn, **kw)

    logits = {}
    for name, backend in (("hip", HipAttention), ("torch", TorchRefFP8Attention)):
        r = fp8_runner(backend, decode_graphs=False, piecewise_graphs=False)
        seqs = [Sequence(list(p)) for p in PROMPTS]
        got = {}
        orig = r.model.logits
        r.model.logits = lambda h, _o=orig, _g=got: _g.setdefault("l", _o(h))
        r.prefill(seqs)
        logits[name] = got["l"]
    scale = logits["torch"].abs().max().item()
    assert (logits["hip"] - logits["torch"]).abs().max().item() <= 0.05 * scale
    runners = [fp8_runner(HipAttention, max_graph_batch=8, decode_graphs=g, piecewise_graphs=False) for g in (True, False)]
    seqs = [[Sequence(list(p)) for p in PROMPTS[:3]] for _ in runners]
    for r, s in zip(runners, seqs):
        r.prefill(s)
    for step in range(4):
        outs = []
        for r, s in zip(runners, seqs):
            got = {}
            orig = r.model.logits
            r.model.logits = lambda h, _o=orig, _g=got: _g.setdefault("l", _o(h))
            r.decode(s)
            r.model.logits = orig
            outs.append(got["l"])
        for g, e in zip(seqs[0], seqs[1]):  # teacher-force the graph runner to the eager tokens
            g.tokens[-1] = e.tokens[-1]
        diff = (outs[0] - outs[1]).abs().max().item()
        assert diff <= 3e-2 * outs[1].abs().max().item(), (step, diff)
    assert runners[0].paths["decode_graph"] == 4
