"""Llama decoder over a flat, paged-KV batch, calling an attention backend.

The layer structure is the reference's (src/kvserve/model.py): tokens of all sequences
packed without padding, fused QKV and gate/up projections, K/V written to and read from
the shared paged pool through `backend.write_kv` / `backend.forward`, and the forward pass
split at the attention calls into num_layers + 1 row-wise pieces (model.py:187-212).
GEMMs, norms and RoPE are PyTorch (hipBLASLt GEMMs on ROCm); attention is the backend's. On
the GPU with 16-bit weights (`fused_ops`), the residual add + RMSNorm and SiLU * up run as
single libkvhip kernels and projections of at most 4 rows as its GEMV, the gate_up one with
SiLU * up in its epilogue (engine/ops.py).
"""

from __future__ import annotations

import math
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

from kvserve_amd.attention import AttentionMetadata, HipAttention
from kvserve_amd.engine import ops
from kvserve_amd.engine.config import ModelConfig


class RMSNorm(nn.Module):
    """x / rms(x) in fp32, cast back, times the weight (model.py:22-32)."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x32 = x.float()
        x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * x32.to(x.dtype)


def rope_inv_freq(cfg: ModelConfig) -> torch.Tensor:
    """Inverse frequencies, with Llama 3's frequency-dependent long-context scaling when the
    config asks for it (model.py:35-52): wavelengths above original_ctx / low_freq_factor are
    divided by `factor`, those below original_ctx / high_freq_factor kept, and the band in
    between interpolated linearly in original_ctx / wavelength."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    sc = cfg.rope_scaling or {}
    if sc.get("rope_type", sc.get("type")) != "llama3":
        return inv
    factor, lo, hi = sc["factor"], sc["low_freq_factor"], sc["high_freq_factor"]
    ctx = sc["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv
    long_wave = wavelen > ctx / lo
    short_wave = wavelen < ctx / hi
    blend = (ctx / wavelen - lo) / (hi - lo)
    mid = (1 - blend) * inv / factor + blend * inv
    return torch.where(long_wave, inv / factor, torch.where(short_wave, inv, mid))


class RotaryEmbedding(nn.Module):
    """cos/sin tables for positions [0, max_positions), fp32; rotate-half convention."""

    def __init__(self, cfg: ModelConfig, max_positions: int, device=None):
        super().__init__()
        freqs = torch.outer(torch.arange(max_positions, dtype=torch.float32), rope_inv_freq(cfg))
        emb = torch.cat([freqs, freqs], dim=-1)
        self.register_buffer("cos", emb.cos().to(device), persistent=False)
        self.register_buffer("sin", emb.sin().to(device), persistent=False)

    def forward(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor):
        cos = self.cos[positions].to(q.dtype)[:, None]  # [T, 1, D]
        sin = self.sin[positions].to(q.dtype)[:, None]
        return q * cos + _rotate_half(q) * sin, k * cos + _rotate_half(k) * sin


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    a, b = x.chunk(2, dim=-1)
    return torch.cat([-b, a], dim=-1)


class Attention(nn.Module):
    def __init__(self, cfg: ModelConfig, backend):
        super().__init__()
        self.backend = backend
        self.num_heads, self.num_kv_heads, self.head_dim = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        self.q_size = cfg.num_heads * cfg.head_dim
        self.kv_size = cfg.num_kv_heads * cfg.head_dim
        self.qkv_proj = nn.Linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, bias=False)
        self.o_proj = nn.Linear(self.q_size, cfg.hidden_size, bias=False)
        self.scale = self.head_dim**-0.5
        # per-layer scales of a float8_e4m3fn KV cache (unused for 16-bit caches)
        self.k_scale = self.v_scale = 1.0

    def _kv_scales(self, cache: torch.Tensor) -> dict:
        return {"k_scale": self.k_scale, "v_scale": self.v_scale} if cache.dtype == torch.float8_e4m3fn else {}

    def project(self, x: torch.Tensor, positions: torch.Tensor, rope: RotaryEmbedding):
        """[T, hidden] -> q [T, H, D], k [T, Hkv, D] (RoPE applied), v [T, Hkv, D] (a strided
        view of the fused projection, as in model.py:84-94)."""
        n = x.shape[0]
        q, k, v = self.qkv_proj(x).split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = q.view(n, self.num_heads, self.head_dim)
        k = k.view(n, self.num_kv_heads, self.head_dim)
        v = v.view(n, self.num_kv_heads, self.head_dim)
        q, k = rope(q, k, positions)
        return q, k, v

    def attend(self, q, k, v, kv_cache: torch.Tensor, meta: AttentionMetadata, out: torch.Tensor | None = None):
        """Write this step's K/V into the paged cache and attend over it (model.py:96-108)."""
        k_cache, v_cache = kv_cache[0], kv_cache[1]
        sc = self._kv_scales(k_cache)
        self.backend.write_kv(k_cache, v_cache, k, v, meta.slot_mapping, **sc)
        return self.backend.forward(q, k_cache, v_cache, meta, self.scale, out=out, **sc)

    def attend_fused(self, qkv, positions, rope: RotaryEmbedding, kv_cache: torch.Tensor, meta: AttentionMetadata,
                     out: torch.Tensor | None = None, h: torch.Tensor | None = None):  # fmt: skip
        """RoPE, QKV split and the cache write in the backend's one kernel, then attention: the
        same result as project() + attend() (bit for bit) with the RoPE moved out of the piece.
        With qkv None the piece stopped before the projection (h, decode-sized batches): the
        backend's gemv_rope_and_cache projects and rotates in the same kernel."""
        k_cache, v_cache = kv_cache[0], kv_cache[1]
        sc = self._kv_scales(k_cache)
        if qkv is None:
            q = self.backend.gemv_rope_and_cache(h, self.qkv_proj.weight, positions, rope.cos, rope.sin, k_cache,
                                                 v_cache, meta.slot_mapping, self.num_heads, **sc)  # fmt: skip
        else:
            q = self.backend.rope_and_cache(qkv, positions, rope.cos, rope.sin, k_cache, v_cache, meta.slot_mapping,
                                            self.num_heads, **sc)  # fmt: skip
        return self.backend.forward(q, k_cache, v_cache, meta, self.scale, out=out, **sc)


class MLP(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.gate_up_proj = nn.Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class DecoderLayer(nn.Module):
    def __init__(self, cfg: ModelConfig, backend):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg, backend)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = MLP(cfg)


# Hugging Face projection name -> (fused parameter, shard)
_FUSED = {
    "q_proj": ("qkv_proj", 0),
    "k_proj": ("qkv_proj", 1),
    "v_proj": ("qkv_proj", 2),
    "gate_proj": ("gate_up_proj", 0),
    "up_proj": ("gate_up_proj", 1),
}


class LlamaForCausalLM(nn.Module):
    def __init__(self, cfg: ModelConfig, max_positions: int, backend=HipAttention):
        super().__init__()
        self.cfg = cfg
        self.max_positions = max_positions
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg, backend) for _ in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight
        self.rope = RotaryEmbedding(cfg, max_positions)
        # a backend with a fused RoPE + cache-write kernel takes the raw QKV projection
        self.fused_rope = bool(getattr(backend, "fused_rope_cache", False))
        self.backend = backend
        # decode-sized batches: the QKV projection fused with RoPE + cache write (fused_ops only)
        self._gemv_rope = hasattr(backend, "gemv_rope_and_cache")
        # libkvhip's fused elementwise kernels and GEMV (set on the GPU, 16-bit weights)
        self.fused_ops = False

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_caches: torch.Tensor,
                meta: AttentionMetadata) -> torch.Tensor:  # fmt: skip
        """Final hidden states [T, hidden]; kv_caches [layers, 2, blocks, block_size, kv_heads, D]."""
        x, q, k, v = self.piece(0, input_ids, positions, None, None)
        for i, layer in enumerate(self.layers):
            if self.fused_rope:
                attn = layer.self_attn.attend_fused(q, positions, self.rope, kv_caches[i], meta, h=k)
            else:
                attn = layer.self_attn.attend(q, k, v, kv_caches[i], meta)
            x, q, k, v = self.piece(i + 1, input_ids, positions, x, attn)
        return x

    def piece(self, i: int, input_ids, positions, x, attn):
        """Everything between attention call i - 1 and attention call i (i = 0 .. num_layers):
        finish layer i - 1 (output projection, residual, MLP), start layer i (norm, QKV, RoPE).
        Row-wise, never touches the KV cache (model.py:187-212). Returns (x, q, k, v), or
        (final hidden states, None, None, None) for the last piece. With a fused-RoPE backend
        the piece stops at the QKV projection: (x, qkv, None, None)."""
        if self.fused_ops:
            return self._piece_fused(i, input_ids, positions, x, attn)
        if i == 0:
            x = self.embed_tokens(input_ids)
        else:
            prev = self.layers[i - 1]
            x = x + prev.self_attn.o_proj(attn.flatten(1))
            x = x + prev.mlp(prev.post_attention_layernorm(x))
        if i == len(self.layers):
            return self.norm(x), None, None, None
        layer = self.layers[i]
        h = layer.input_layernorm(x)
        if self.fused_rope:
            return x, layer.self_attn.qkv_proj(h), None, None
        q, k, v = layer.self_attn.project(h, positions, self.rope)
        return x, q, k, v

    def _piece_fused(self, i: int, input_ids, positions, x, attn):
        """piece() with libkvhip's kernels: the same operations, the residual adds fused into
        the following norm, SiLU * up in one pass and small-batch projections on the GEMV."""
        n = len(self.layers)
        if i == 0:
            x, h = ops.add_rmsnorm(self.embed_tokens(input_ids), None, self.layers[0].input_layernorm.weight,
                                   self.layers[0].input_layernorm.eps)  # fmt: skip
        else:
            prev = self.layers[i - 1]
            o = ops.linear(attn.flatten(1), prev.self_attn.o_proj.weight)
            x, h = ops.add_rmsnorm(x, o, prev.post_attention_layernorm.weight, prev.post_attention_layernorm.eps)
            d = ops.linear(ops.mlp_act(h, prev.mlp.gate_up_proj.weight), prev.mlp.down_proj.weight)
            norm = self.norm if i == n else self.layers[i].input_layernorm
            x, h = ops.add_rmsnorm(x, d, norm.weight, norm.eps)
            if i == n:
                return h, None, None, None
        layer = self.layers[i]
        if self.fused_rope and self._gemv_rope and ops.qkv_rope_fused(h.shape[0], *layer.self_attn.qkv_proj.weight.shape):
            return x, None, h, None  # the projection runs in the attention step (gemv_rope_and_cache)
        qkv = ops.linear(h, layer.self_attn.qkv_proj.weight)
        if self.fused_rope:
            return x, qkv, None, None
        q, k, v = qkv.split([layer.self_attn.q_size, layer.self_attn.kv_size, layer.self_attn.kv_size], dim=-1)
        q = q.view(-1, layer.self_attn.num_heads, layer.self_attn.head_dim)
        k = k.view(-1, layer.self_attn.num_kv_heads, layer.self_attn.head_dim)
        v = v.view(-1, layer.self_attn.num_kv_heads, layer.self_attn.head_dim)
        q, k = self.rope(q, k, positions)
        return x, q, k, v

    @torch.inference_mode()
    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.fused_ops:
            return ops.linear(hidden, self.lm_head.weight).float()
        return self.lm_head(hidden).float()

    # -- weights ----------------------------------------------------------------------------
    def _shard_range(self, target: str, shard: int) -> tuple[int, int]:
        c = self.cfg
        if target == "qkv_proj":
            q, kv = c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim
            return [(0, q), (q, kv), (q + kv, kv)][shard]
        return shard * c.intermediate_size, c.intermediate_size

    @torch.inference_mode()
    def load_weights(self, path: Path) -> None:
        """Load Hugging Face safetensors (model.layers.N.self_attn.q_proj.weight, ...) into the
        fused parameters."""
        from safetensors import safe_open

        params = dict(self.named_parameters())
        loaded: set[str] = set()
        for file in sorted(Path(path).glob("*.safetensors")):
            with safe_open(str(file), framework="pt") as f:
                for hf_name in f.keys():  # noqa: SIM118
                    name = hf_name.removeprefix("model.")
                    module, _, leaf = name.rpartition(".")
                    parent, _, proj = module.rpartition(".")
                    t = f.get_tensor(hf_name)
                    if proj in _FUSED:
                        target, shard = _FUSED[proj]
                        name = f"{parent}.{target}.{leaf}"
                        off, size = self._shard_range(target, shard)
                        params[name].data[off : off + size].copy_(t)
                    else:
                        if name == "lm_head.weight" and self.cfg.tie_word_embeddings:
                            continue
                        params[name].data.copy_(t)
                    loaded.add(name)
        missing = set(params) - loaded - ({"lm_head.weight"} if self.cfg.tie_word_embeddings else set())
        if missing:
            raise ValueError(f"weights missing from checkpoint: {sorted(missing)[:5]}")

    @torch.inference_mode()
    def init_random(self, seed: int, std: float = 0.02) -> None:
        """Synthetic weights in place (no checkpoint): N(0, std) projections and embeddings,
        norm weights 1. Drawn on the parameters' own device so large models fill quickly."""
        dev = next(self.parameters()).device
        gen = torch.Generator(device=dev).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("layernorm.weight") or name == "norm.weight":
                p.fill_(1.0)
            else:
                p.copy_(torch.randn(p.shape, generator=gen, device=dev, dtype=torch.float32).to(p.dtype) * std)


def build_model(cfg: ModelConfig, device, dtype: torch.dtype, max_positions: int, backend=HipAttention,
                weights: Path | None = None, seed: int = 0, std: float = 0.02,
                fused_ops: bool | None = None) -> LlamaForCausalLM:  # fmt: skip
    """Model on `device` in `dtype`: weights from a safetensors directory, else synthetic.
    fused_ops (default: on a GPU with 16-bit weights) selects libkvhip's layer kernels."""
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg, max_positions, backend)
    model = model.to(dtype).to_empty(device=device)  # never materialise fp32 weights
    if cfg.tie_word_embeddings:
        model.lm_head.weight = model.embed_tokens.weight
    if weights is not None:
        model.load_weights(weights)
    else:
        model.init_random(seed, std)
    model.rope = RotaryEmbedding(cfg, max_positions, device=device)  # fp32 tables, after the cast
    probe = torch.empty(0, dtype=dtype, device=device)
    model.fused_ops = ops.enabled(probe) if fused_ops is None else bool(fused_ops)
    if model.fused_ops and not ops.enabled(probe):
        raise ValueError("fused_ops needs a GPU and fp16 / bf16 weights")
    return model.eval()
