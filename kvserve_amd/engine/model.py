"""Paged Llama decoder used to drive the attention backend as kvserve's model drives it.

Layout of the computation. A step's tokens (every sequence's, packed without padding) flow
through `num_layers + 1` *stages* separated by `num_layers` *attention steps*:

    stage 0        embed -> norm -> fused QKV projection of layer 0
    attention i    RoPE(q, k), K/V into the paged cache, paged attention       (backend)
    stage i + 1    o_proj -> residual -> norm -> gate_up -> SiLU * up -> down -> residual
                   -> norm -> fused QKV projection of layer i + 1  (final norm for the last)

Stages are row-wise over the flat batch and never touch the KV cache, so they can be
replayed from HIP graphs captured at a padded token count while the attention steps run on
the real tokens with the step's own metadata (kvserve's piecewise boundary,
src/kvserve/cuda_graph.py:140-241). Ending a stage at the *unrotated* projection puts RoPE
on the attention side of the boundary, where the HIP backend applies it in the same kernel
that writes the cache (`HipAttention.rope_and_cache`); backends without that kernel get the
split + RoPE + `write_kv` sequence of the reference's `Attention.project` / `attend`
(src/kvserve/model.py:84-108).

Weights are plain tensors per layer (`LayerWeights`), the projections fused as the
reference fuses them (q|k|v rows, gate|up rows). The arithmetic is Hugging Face Llama's
(RMSNorm with fp32 statistics, rotate-half RoPE with Llama 3 frequency scaling, SiLU MLP),
which the CPU tests pin against transformers' own model. On the GPU with 16-bit weights the
row-wise work runs on libkvhip's layer kernels (`engine.ops`).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import NamedTuple

import torch
import torch.nn.functional as F

from kvserve_amd.attention import AttentionMetadata, HipAttention
from kvserve_amd.engine import ops
from kvserve_amd.engine.config import ModelConfig

# -- arithmetic ------------------------------------------------------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """weight * (x / sqrt(mean(x^2) + eps)), statistics in fp32, normalised rows rounded to
    x's dtype before the weight multiplies them (Llama's RMSNorm; reference model.py:22-32)."""
    xf = x.float()
    inv_rms = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return weight * (xf * inv_rms).to(x.dtype)


def rope_inv_freq(cfg: ModelConfig) -> torch.Tensor:
    """RoPE inverse frequencies theta^(-2i/D), i < D/2, with Llama 3's long-context rescaling
    when the config carries it (reference model.py:35-52): a component whose wavelength
    2 pi / f exceeds original_ctx / low_freq_factor is slowed by `factor`, one below
    original_ctx / high_freq_factor is kept, and in between the two are blended linearly in
    original_ctx / wavelength."""
    half = torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float()
    base = 1.0 / (cfg.rope_theta ** (half / cfg.head_dim))
    sc = cfg.rope_scaling or {}
    if sc.get("rope_type", sc.get("type")) != "llama3":
        return base
    ctx = sc["original_max_position_embeddings"]
    lo, hi, factor = sc["low_freq_factor"], sc["high_freq_factor"], sc["factor"]
    wavelength = 2 * math.pi / base
    t = (ctx / wavelength - lo) / (hi - lo)  # 0 at the long-wave edge, 1 at the short-wave edge
    blended = (1 - t) * base / factor + t * base
    out = torch.where(wavelength < ctx / hi, base, blended)
    return torch.where(wavelength > ctx / lo, base / factor, out)


def rope_tables(cfg: ModelConfig, max_positions: int, device=None) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos / sin tables [max_positions, head_dim]: angle p * f_i in both halves of a row."""
    angles = torch.arange(max_positions, dtype=torch.float32)[:, None] * rope_inv_freq(cfg)[None, :]
    angles = angles.repeat(1, 2)
    return angles.cos().to(device), angles.sin().to(device)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [T, heads, D] rotated by per-token cos / sin rows [T, D] (already in x's dtype):
    x * cos + (-x2, x1) * sin with x1, x2 the two halves of the last dim."""
    d = x.shape[-1] // 2
    turned = torch.cat((-x[..., d:], x[..., :d]), dim=-1)
    return x * cos[:, None, :] + turned * sin[:, None, :]


# -- weights ---------------------------------------------------------------------------------


@dataclass
class LayerWeights:
    attn_norm: torch.Tensor  # [hidden]
    wqkv: torch.Tensor  # [(H + 2 Hkv) D, hidden]: query heads, then key heads, then value heads
    wo: torch.Tensor  # [hidden, H D]
    mlp_norm: torch.Tensor  # [hidden]
    w_gate_up: torch.Tensor  # [2 I, hidden]: gate rows, then up rows
    w_down: torch.Tensor  # [hidden, I]
    k_scale: float = 1.0  # per-layer scales of a float8_e4m3fn KV cache
    v_scale: float = 1.0


@dataclass
class Weights:
    embed: torch.Tensor  # [vocab, hidden]
    layers: list[LayerWeights] = field(default_factory=list)
    final_norm: torch.Tensor | None = None
    lm_head: torch.Tensor | None = None  # the embedding itself when tied


def random_weights(cfg: ModelConfig, device, dtype: torch.dtype, seed: int = 0, std: float = 0.02) -> Weights:
    """Synthetic weights of the model's shape: N(0, std) matrices drawn on `device` from one
    seeded generator (in a fixed order), norm weights 1."""
    gen = torch.Generator(device=device).manual_seed(seed)

    def normal(*shape: int) -> torch.Tensor:
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    def ones() -> torch.Tensor:
        return torch.ones(cfg.hidden_size, device=device, dtype=dtype)

    H, Hkv, D, hid, inter = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size, cfg.intermediate_size
    w = Weights(embed=normal(cfg.vocab_size, hid))
    for _ in range(cfg.num_layers):
        w.layers.append(LayerWeights(ones(), normal((H + 2 * Hkv) * D, hid), normal(hid, H * D), ones(),
                                     normal(2 * inter, hid), normal(hid, inter)))  # fmt: skip
    w.final_norm = ones()
    w.lm_head = w.embed if cfg.tie_word_embeddings else normal(cfg.vocab_size, hid)
    return w


def load_hf_weights(path: Path, cfg: ModelConfig, device, dtype: torch.dtype) -> Weights:
    """Weights from a Hugging Face Llama checkpoint (*.safetensors under `path`), with the
    separate q/k/v and gate/up matrices concatenated row-wise into the fused projections."""
    from safetensors import safe_open

    files = sorted(Path(path).glob("*.safetensors"))
    where: dict[str, Path] = {}
    for f in files:
        with safe_open(str(f), framework="pt") as h:
            for name in h.keys():  # noqa: SIM118  (a safetensors handle, not a mapping)
                where[name] = f

    def get(name: str) -> torch.Tensor:
        for key in (name, f"model.{name}"):
            if key in where:
                with safe_open(str(where[key]), framework="pt") as h:
                    return h.get_tensor(key).to(device=device, dtype=dtype)
        raise KeyError(f"{path}: checkpoint has no tensor {name!r}")

    w = Weights(embed=get("embed_tokens.weight"))
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        qkv = torch.cat([get(p + f"self_attn.{x}_proj.weight") for x in "qkv"])
        gate_up = torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")])
        w.layers.append(LayerWeights(get(p + "input_layernorm.weight"), qkv, get(p + "self_attn.o_proj.weight"),
                                     get(p + "post_attention_layernorm.weight"), gate_up,
                                     get(p + "mlp.down_proj.weight")))  # fmt: skip
    w.final_norm = get("norm.weight")
    w.lm_head = w.embed if cfg.tie_word_embeddings else get("lm_head.weight")
    return w


# -- the model -------------------------------------------------------------------------------


class StageOut(NamedTuple):
    """What a stage hands to the next attention step (or, after the last stage, the final
    hidden states in `resid`). Exactly one of `qkv` / `normed` is set before an attention step:
    `normed` when the projection is deferred into the attention step's fused kernel."""

    resid: torch.Tensor  # [T, hidden] residual stream
    qkv: torch.Tensor | None  # [T, (H + 2 Hkv) D] fused projection, not yet rotated
    normed: torch.Tensor | None  # [T, hidden] the layer's normalised input


class PagedLlama:
    """A Llama decoder over the flat paged batch, calling an attention backend with kvserve's
    interface (`write_kv` / `forward`, src/kvserve/attention.py:39-102)."""

    def __init__(self, cfg: ModelConfig, weights: Weights, backend=HipAttention, max_positions: int = 4096,
                 fused_ops: bool | None = None, fused_rope: bool | None = None):  # fmt: skip
        self.cfg = cfg
        self.w = weights
        self.backend = backend
        self.device, self.dtype = weights.embed.device, weights.embed.dtype
        self.max_positions = max_positions
        self.cos, self.sin = rope_tables(cfg, max_positions, self.device)
        self.scale = cfg.head_dim**-0.5
        self.q_width = cfg.num_heads * cfg.head_dim
        self.kv_width = cfg.num_kv_heads * cfg.head_dim
        # What the backend offers beyond write_kv / forward. fused_rope=False drives it exactly
        # as kvserve's Attention.attend does (src/kvserve/model.py:84-108): split + RoPE in
        # torch, write_kv with v a strided view of the fused QKV output, then forward(out=...).
        offered = callable(getattr(backend, "rope_and_cache", None))
        if fused_rope and not offered:
            raise ValueError("the backend has no fused RoPE + cache write (rope_and_cache)")
        self.fused_rope = offered if fused_rope is None else bool(fused_rope)
        self.fused_projection = self.fused_rope and callable(getattr(backend, "gemv_rope_and_cache", None))
        probe = torch.empty(0, dtype=self.dtype, device=self.device)
        self.fused_ops = ops.enabled(probe) if fused_ops is None else bool(fused_ops)
        if self.fused_ops and not ops.enabled(probe):
            raise ValueError("libkvhip layer kernels need a GPU and fp16 / bf16 weights")

    @property
    def num_layers(self) -> int:
        return len(self.w.layers)

    # -- row-wise stages ------------------------------------------------------------------------
    def _linear(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        return ops.linear(x, w) if self.fused_ops else F.linear(x, w)

    def _add_norm(self, x: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor):
        """(x + delta, RMSNorm(x + delta)); delta None: (x, RMSNorm(x))."""
        eps = self.cfg.rms_norm_eps
        if self.fused_ops:
            return ops.add_rmsnorm(x, delta, weight, eps)
        if delta is not None:
            x = x + delta
        return x, rms_norm(x, weight, eps)

    def _mlp(self, h: torch.Tensor, lw: LayerWeights) -> torch.Tensor:
        if self.fused_ops:
            return ops.linear(ops.mlp_act(h, lw.w_gate_up), lw.w_down)
        gate, up = F.linear(h, lw.w_gate_up).chunk(2, dim=-1)
        return F.linear(F.silu(gate) * up, lw.w_down)

    def defers_projection(self, rows: int) -> bool:
        """Whether a layer's QKV projection over `rows` rows moves into the attention step
        (the backend's projection + RoPE + cache-write kernel, decode-sized batches only)."""
        if not (self.fused_ops and self.fused_rope and self.fused_projection):
            return False
        return ops.qkv_rope_fused(rows, *self.w.layers[0].wqkv.shape)

    def stage(self, i: int, input_ids: torch.Tensor | None, resid: torch.Tensor | None, attn: torch.Tensor | None,
              defer: bool = False) -> StageOut:  # fmt: skip
        """Stage i of num_layers + 1 (see the module docstring). Stage 0 reads `input_ids`; a
        later stage reads the residual stream and layer i - 1's attention output [T, H, D].
        `defer` leaves the next projection to the attention step (`defers_projection`)."""
        L = self.num_layers
        if i == 0:
            x, h = self._add_norm(F.embedding(input_ids, self.w.embed), None, self.w.layers[0].attn_norm)
        else:
            prev = self.w.layers[i - 1]
            o = self._linear(attn.flatten(1), prev.wo)
            x, h = self._add_norm(resid, o, prev.mlp_norm)
            nxt = self.w.final_norm if i == L else self.w.layers[i].attn_norm
            x, h = self._add_norm(x, self._mlp(h, prev), nxt)
            if i == L:
                return StageOut(h, None, None)
        if defer:
            return StageOut(x, None, h)
        return StageOut(x, self._linear(h, self.w.layers[i].wqkv), None)

    # -- attention steps -----------------------------------------------------------------------
    def attention(self, i: int, s: StageOut, positions: torch.Tensor, kv_layer: torch.Tensor, meta: AttentionMetadata,
                  out: torch.Tensor | None = None, q_out: torch.Tensor | None = None) -> torch.Tensor:  # fmt: skip
        """Layer i's attention over the pool slice kv_layer [2, blocks, BS, Hkv, D]: RoPE, this
        step's K/V into the cache at meta.slot_mapping, then paged attention -> [T, H, D] (into
        `out` if given; `q_out` receives the rotated queries on the fused paths)."""
        lw = self.w.layers[i]
        k_cache, v_cache = kv_layer[0], kv_layer[1]
        sc = {"k_scale": lw.k_scale, "v_scale": lw.v_scale} if k_cache.dtype == torch.float8_e4m3fn else {}
        H = self.cfg.num_heads
        b = self.backend
        if s.normed is not None:
            q = b.gemv_rope_and_cache(s.normed, lw.wqkv, positions, self.cos, self.sin, k_cache, v_cache,
                                      meta.slot_mapping, H, out=q_out, **sc)  # fmt: skip
        elif self.fused_rope:
            q = b.rope_and_cache(s.qkv, positions, self.cos, self.sin, k_cache, v_cache, meta.slot_mapping, H,
                                 out=q_out, **sc)  # fmt: skip
        else:
            n, D = s.qkv.shape[0], self.cfg.head_dim
            q, k, v = s.qkv.split([self.q_width, self.kv_width, self.kv_width], dim=-1)
            cos, sin = self.cos[positions].to(q.dtype), self.sin[positions].to(q.dtype)
            q = apply_rope(q.view(n, H, D), cos, sin)
            k = apply_rope(k.view(n, -1, D), cos, sin)
            b.write_kv(k_cache, v_cache, k, v.view(n, -1, D), meta.slot_mapping, **sc)
        return b.forward(q, k_cache, v_cache, meta, self.scale, out=out, **sc)

    # -- whole passes ----------------------------------------------------------------------------
    @torch.inference_mode()
    def hidden_states(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_caches: torch.Tensor,
                      meta: AttentionMetadata) -> torch.Tensor:  # fmt: skip
        """Final hidden states [T, hidden] of one step; kv_caches [L, 2, blocks, BS, Hkv, D]."""
        defer = self.defers_projection(input_ids.shape[0])
        s = self.stage(0, input_ids, None, None, defer)
        for i in range(self.num_layers):
            a = self.attention(i, s, positions, kv_caches[i], meta)
            s = self.stage(i + 1, None, s.resid, a, defer)
        return s.resid

    __call__ = hidden_states

    @torch.inference_mode()
    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """fp32 logits [T, vocab]."""
        return self._linear(hidden, self.w.lm_head).float()


def build_model(cfg: ModelConfig, device, dtype: torch.dtype, max_positions: int, backend=HipAttention,
                weights: Path | None = None, seed: int = 0, std: float = 0.02,
                fused_ops: bool | None = None, fused_rope: bool | None = None) -> PagedLlama:  # fmt: skip
    """A PagedLlama on `device` in `dtype`: weights from a Hugging Face safetensors directory,
    else synthetic (`random_weights`). fused_ops (default: on a GPU with 16-bit weights) selects
    libkvhip's layer kernels for the row-wise work; fused_rope=False keeps the backend to
    kvserve's write_kv + forward calls (default: its fused RoPE + cache write when offered)."""
    device = torch.device(device)
    w = load_hf_weights(weights, cfg, device, dtype) if weights is not None else random_weights(cfg, device, dtype,
                                                                                                 seed, std)  # fmt: skip
    return PagedLlama(cfg, w, backend, max_positions, fused_ops, fused_rope)
