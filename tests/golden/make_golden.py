"""Writes tests/golden/fixtures.npz: small paged batches and their fp64 oracle outputs.

    python -m tests.golden.make_golden

Inputs are N(0, 1) rounded to bf16 (stored as raw bf16 bits), so the GPU kernels consume
exactly the values the oracle saw. Outputs come from the plain-C fp64 oracle
(oracle/paged_attention_oracle.c). The reference ships no golden vectors for this path;
these pin the oracle against regressions and give the GPU tests fixed expected values.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
FIXTURES = HERE / "fixtures.npz"

# (name, query_lens, context_lens, H, Hkv, D, BS)
SPECS = [
    ("decode_gqa", [1, 1, 1, 1], [5, 17, 64, 100], 4, 1, 64, 16),
    ("chunked_prefill", [50, 16, 3], [100, 16, 250], 2, 1, 64, 16),
    ("mixed_mha", [1, 1, 37, 1], [40, 211, 0, 2], 2, 2, 64, 16),
    ("verify_d128_bs32", [5, 5], [70, 33], 4, 2, 128, 32),
]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bits_to_f64(b: np.ndarray) -> np.ndarray:
    return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(torch.float64).numpy()


def build_fixtures() -> dict[str, dict[str, np.ndarray]]:
    import oracle
    from kvserve_amd import workloads

    out = {}
    for i, (name, ql, cl, H, Hkv, D, BS) in enumerate(SPECS):
        w = workloads.custom(name, ql, cl, H, Hkv, D, BS, seed=100 + i)
        rng = np.random.default_rng(100 + i)
        q = bf16_bits(rng.standard_normal((w.num_tokens, H, D)))
        kc = bf16_bits(rng.standard_normal((w.num_blocks, BS, Hkv, D)))
        vc = bf16_bits(rng.standard_normal((w.num_blocks, BS, Hkv, D)))
        bt = np.zeros((len(ql), w.table_width()), dtype=np.int64)
        for s, t in enumerate(w.tables):
            bt[s, : len(t)] = t
        sl = np.asarray(w.seq_lens, dtype=np.int64)
        qsl = np.concatenate([[0], np.cumsum(ql)]).astype(np.int64)
        scale = np.float64(D**-0.5)
        res = oracle.paged_attention_f64(bits_to_f64(q), bits_to_f64(kc), bits_to_f64(vc), bt, sl, qsl, float(scale))
        out[name] = dict(q_bits=q, k_bits=kc, v_bits=vc, block_tables=bt, seq_lens=sl, query_start_loc=qsl,
                         scale=scale, out=res)  # fmt: skip
    return out


def load_fixtures() -> dict[str, dict[str, np.ndarray]]:
    """Fixtures keyed by name; adds float64 views q / k_cache / v_cache of the bf16 bits."""
    raw = np.load(FIXTURES, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in raw.files})
    res = {}
    for n in names:
        fx = {k.split("/", 1)[1]: raw[k] for k in raw.files if k.startswith(n + "/")}
        fx["q"] = bits_to_f64(fx["q_bits"])
        fx["k_cache"] = bits_to_f64(fx["k_bits"])
        fx["v_cache"] = bits_to_f64(fx["v_bits"])
        res[n] = fx
    return res


def main() -> None:
    fx = build_fixtures()
    flat = {f"{n}/{k}": v for n, d in fx.items() for k, v in d.items()}
    np.savez_compressed(FIXTURES, **flat)
    print(FIXTURES, FIXTURES.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
