"""Pins the CPU oracle before anything is compared against it (CPU only).

The reference ships no golden vectors for this path, so the oracle is pinned by
  * agreement of two independent restatements: the plain-C fp64 brute force and the
    torch restatement of TorchAttention.forward (src/kvserve/attention.py:47-82);
  * known answers the mathematics fixes (single key, constant V, zero query, two-key
    softmax in closed form, logical-page identity);
  * invariances (score shift, physical block permutation, table padding width, GQA
    expansion to MHA);
  * the reference's own slot test (tests/test_kv_cache.py:57-63);
and each planted mistake (oracle.MUTANTS) must fail at least one of these checks.
"""

import math
import random

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_reference
from kvserve_amd import workloads

# ------------------------------------------------------------------------------------
# helpers


def make_np_batch(query_lens, context_lens, H, Hkv, D, BS, seed=0, spare=8, width_extra=0):
    w = workloads.custom("t", query_lens, context_lens, H, Hkv, D, BS, seed=seed, spare_blocks=spare)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((w.num_tokens, H, D))
    kc = rng.standard_normal((w.num_blocks, BS, Hkv, D))
    vc = rng.standard_normal((w.num_blocks, BS, Hkv, D))
    width = w.table_width() + width_extra
    bt = np.zeros((len(w.tables), width), dtype=np.int64)
    for i, t in enumerate(w.tables):
        bt[i, : len(t)] = t
    sl = np.asarray(w.seq_lens, dtype=np.int64)
    qsl = np.concatenate([[0], np.cumsum(query_lens)]).astype(np.int64)
    return dict(q=q, kc=kc, vc=vc, bt=bt, sl=sl, qsl=qsl, ql=np.asarray(query_lens), scale=D**-0.5, w=w)


def c_attn(flags=0):
    def f(q, kc, vc, bt, sl, qsl, scale):
        return oracle.paged_attention_f64(q, kc, vc, bt, sl, qsl, scale, flags)

    return f


def torch_attn(q, kc, vc, bt, sl, qsl, scale):
    ql = np.diff(qsl)
    out = torch_reference.forward(
        torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc), torch.from_numpy(bt),
        torch.from_numpy(sl), torch.from_numpy(ql), scale,
    )  # fmt: skip
    return out.numpy()


def run(attn, b):
    return attn(b["q"], b["kc"], b["vc"], b["bt"], b["sl"], b["qsl"], b["scale"])


# ------------------------------------------------------------------------------------
# pinning checks; each returns True when the implementation passes


def check_single_key(attn):
    """seq_len = 1: the one visible key gets weight 1, out = v0."""
    b = make_np_batch([1, 1], [0, 0], 4, 2, 8, 4, seed=1)
    out = run(attn, b)
    for s in range(2):
        blk = b["bt"][s, 0]
        for h in range(4):
            if not np.allclose(out[s, h], b["vc"][blk, 0, h // 2], atol=1e-12):
                return False
    return True


def check_constant_v(attn):
    """V identical for every key of a kv head -> out = that V."""
    b = make_np_batch([3, 1, 5], [6, 9, 0], 4, 2, 8, 4, seed=2)
    vrow = np.random.default_rng(3).standard_normal((2, 8))
    b["vc"][:] = vrow[None, None]
    out = run(attn, b)
    return all(np.allclose(out[:, h], vrow[h // 2][None], atol=1e-12) for h in range(4))


def check_zero_query_mean(attn):
    """q = 0 -> uniform weights -> mean of the visible V rows (ctx + i + 1 of them)."""
    ql, cl = [2, 1, 4], [5, 0, 7]
    b = make_np_batch(ql, cl, 4, 2, 8, 4, seed=4)
    b["q"][:] = 0.0
    out = run(attn, b)
    BS = 4
    for s, (n, c) in enumerate(zip(ql, cl)):
        for i in range(n):
            t = b["qsl"][s] + i
            keys = range(c + i + 1)
            for h in range(4):
                rows = [b["vc"][b["bt"][s, j // BS], j % BS, h // 2] for j in keys]
                if not np.allclose(out[t, h], np.mean(rows, axis=0), atol=1e-12):
                    return False
    return True


def check_two_key_softmax(attn):
    """Two keys, V = one-hot: out[0] = softmax(scale * [a, b])[0] in closed form."""
    D, BS = 8, 4
    b = make_np_batch([1], [1], 1, 1, D, BS, seed=5)
    rng = np.random.default_rng(6)
    q = rng.standard_normal(D)
    k0, k1 = rng.standard_normal(D), rng.standard_normal(D)
    blk = b["bt"][0, 0]
    b["q"][0, 0] = q
    b["kc"][blk, 0, 0], b["kc"][blk, 1, 0] = k0, k1
    b["vc"][blk, 0, 0] = np.eye(D)[0]
    b["vc"][blk, 1, 0] = np.eye(D)[1]
    sc = b["scale"]
    a, bb = sc * q @ k0, sc * q @ k1
    p0 = 1.0 / (1.0 + math.exp(bb - a))
    out = run(attn, b)[0, 0]
    return np.allclose(out[:2], [p0, 1 - p0], atol=1e-12) and np.allclose(out[2:], 0, atol=1e-12)


def check_page_identity(attn):
    """K = 0 (uniform weights), V[slot] = logical page index of the key stored there:
    out = mean(j // BS for visible j). Catches reading the wrong page of the table."""
    ql, cl, BS = [1, 3], [37, 20], 4
    b = make_np_batch(ql, cl, 2, 1, 4, BS, seed=7)
    b["kc"][:] = 0.0
    b["vc"][:] = -1.0
    for s, t in enumerate(b["w"].tables):
        for p, blk in enumerate(t):
            b["vc"][blk] = p
    out = run(attn, b)
    for s, (n, c) in enumerate(zip(ql, cl)):
        for i in range(n):
            want = np.mean([j // BS for j in range(c + i + 1)])
            if not np.allclose(out[b["qsl"][s] + i], want, atol=1e-12):
                return False
    return True


def check_shift_invariance(attn):
    """Adding the same vector u to every key adds scale*q.u to a row's scores: no change.
    A large u (scores ~ 1e3) also demands the max-shifted softmax."""
    b = make_np_batch([2, 1], [9, 30], 4, 2, 8, 4, seed=8)
    base = run(attn, b)
    u = 400.0 * np.sign(b["q"][0, 0])  # large, same for every key and head
    b2 = dict(b)
    b2["kc"] = b["kc"] + u
    with np.errstate(all="ignore"):
        shifted = run(attn, b2)
    return bool(np.all(np.isfinite(shifted))) and np.allclose(base, shifted, atol=1e-8)


def check_block_permutation(attn):
    """Permuting physical blocks (and rewriting the tables) leaves the output unchanged."""
    b = make_np_batch([1, 4, 1], [14, 3, 22], 4, 2, 8, 4, seed=9)
    base = run(attn, b)
    nb = b["kc"].shape[0]
    perm = np.random.default_rng(10).permutation(nb)  # new id of old block i = perm[i]
    kc, vc = np.empty_like(b["kc"]), np.empty_like(b["vc"])
    kc[perm], vc[perm] = b["kc"], b["vc"]
    b2 = dict(b, kc=kc, vc=vc, bt=perm[b["bt"]])
    return np.allclose(base, run(attn, b2), atol=1e-12)


def check_padding_width(attn):
    """Extra table columns (and stale ids past ceil(seq_len / BS)) are never read."""
    b = make_np_batch([1, 2], [10, 5], 4, 2, 8, 4, seed=11)
    base = run(attn, b)
    bt = np.full((2, b["bt"].shape[1] + 5), 0, dtype=np.int64)
    bt[:, : b["bt"].shape[1]] = b["bt"]
    for s in range(2):
        used = -(-int(b["sl"][s]) // 4)
        bt[s, used:] = np.random.default_rng(12 + s).integers(0, b["kc"].shape[0], bt.shape[1] - used)
    return np.allclose(base, run(attn, dict(b, bt=bt)), atol=1e-12)


def check_gqa_expansion(attn):
    """GQA (H=8, Hkv=2) equals MHA over the cache with each kv head repeated G times."""
    b = make_np_batch([3, 1], [6, 11], 8, 2, 8, 4, seed=13)
    gqa = run(attn, b)
    kc = np.repeat(b["kc"], 4, axis=2)
    vc = np.repeat(b["vc"], 4, axis=2)
    mha = run(attn, dict(b, kc=kc, vc=vc))
    return np.allclose(gqa, mha, atol=1e-12)


def check_matches_torch_reference(attn):
    """Agreement with the torch restatement of TorchAttention.forward on the reference's CASES."""
    for name, (ql, cl) in workloads.REFERENCE_CASES.items():
        for H, Hkv in ((8, 2), (4, 4), (8, 1)):
            b = make_np_batch(ql, cl, H, Hkv, 16, 16, seed=14)
            if not np.allclose(run(attn, b), run(torch_attn, b), atol=1e-10):
                return False
    return True


CHECKS = [
    check_single_key,
    check_constant_v,
    check_zero_query_mean,
    check_two_key_softmax,
    check_page_identity,
    check_shift_invariance,
    check_block_permutation,
    check_padding_width,
    check_gqa_expansion,
    check_matches_torch_reference,
]


# ------------------------------------------------------------------------------------


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_c_oracle_passes(check):
    assert check(c_attn(0))


@pytest.mark.parametrize(
    "check", [c for c in CHECKS if c is not check_matches_torch_reference], ids=lambda c: c.__name__
)
def test_torch_reference_passes(check):
    assert check(torch_attn)


@pytest.mark.parametrize("mutant", sorted(oracle.MUTANTS))
def test_every_planted_mistake_is_caught(mutant):
    attn = c_attn(oracle.MUTANTS[mutant])
    failed = []
    for check in CHECKS:
        try:
            ok = check(attn)
        except (ValueError, FloatingPointError):
            ok = False
        if not ok:
            failed.append(check.__name__)
    assert failed, f"mutant {mutant} passes every pinning check"


def test_head_dim_128_block_32_cross_check():
    """The reference's extra case (tests/test_triton_attention.py:79-86) at fp64."""
    b = make_np_batch([1, 9, 1], [80, 40, 1000], 32, 8, 128, 32, seed=0)
    np.testing.assert_allclose(run(c_attn(0), b), run(torch_attn, b), atol=1e-10)


# ------------------------------------------------------------------------------------
# slot formula and write_kv


@pytest.mark.parametrize(("start", "n"), [(0, 1), (0, 4), (3, 1), (3, 6), (2, 13), (8, 4), (5, 0)])
def test_slots_matches_per_token_slot(start, n):
    """The reference's own check (tests/test_kv_cache.py:57-63): a 20-token sequence in
    4-token blocks allocated [0..4] from a fresh pool, table reversed."""
    table = [4, 3, 2, 1, 0]
    per_token = [table[p // 4] * 4 + p % 4 for p in range(start, start + n)]
    assert oracle.slots(table, 4, start, n) == per_token
    assert workloads.slots_for(table, 4, start, n) == per_token


def test_slots_random_tables():
    rng = random.Random(0)
    for _ in range(200):
        bs = rng.choice([1, 4, 16, 32])
        table = rng.sample(range(1000), 12)
        start = rng.randrange(0, 12 * bs)
        n = rng.randrange(0, 12 * bs - start + 1)
        assert oracle.slots(table, bs, start, n) == workloads.slots_for(table, bs, start, n)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint16])
def test_reshape_and_cache_oracle(dtype):
    """C write vs torch index_put restatement vs the closed form, bitwise."""
    rng = np.random.default_rng(0)
    NB, BS, Hkv, D, T = 9, 4, 2, 8, 13
    slots = rng.choice(NB * BS, size=T, replace=False).astype(np.int64)
    slots[3] = -1  # skipped
    slots[7] = NB * BS + 5  # skipped
    k = rng.integers(0, 2**16, size=(T, Hkv, D)).astype(np.uint16).view(np.uint16)
    v = rng.integers(0, 2**16, size=(T, Hkv, D)).astype(np.uint16)
    if dtype is np.float32:
        k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
        v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    elif dtype is np.float16:
        k, v = k.view(np.float16), v.view(np.float16)
    kc0 = rng.integers(0, 2**16, size=(NB, BS, Hkv, D)).astype(np.uint16)
    if dtype is np.float32:
        kc0 = rng.standard_normal((NB, BS, Hkv, D)).astype(np.float32)
    elif dtype is np.float16:
        kc0 = kc0.view(np.float16)
    kc, vc = kc0.copy(), kc0.copy()
    oracle.reshape_and_cache(k, v, slots, kc, vc)
    valid = (slots >= 0) & (slots < NB * BS)
    flat_k, flat_v = kc.reshape(-1, Hkv, D), vc.reshape(-1, Hkv, D)
    for t in range(T):
        if valid[t]:
            assert flat_k[slots[t]].tobytes() == k[t].tobytes()
            assert flat_v[slots[t]].tobytes() == v[t].tobytes()
    untouched = np.setdiff1d(np.arange(NB * BS), slots[valid])
    assert flat_k[untouched].tobytes() == kc0.reshape(-1, Hkv, D)[untouched].tobytes()
    assert flat_v[untouched].tobytes() == kc0.reshape(-1, Hkv, D)[untouched].tobytes()
    # torch restatement (index_put) on the valid rows agrees bitwise
    if dtype is not np.uint16:
        tk, tv = torch.from_numpy(kc0.copy()), torch.from_numpy(kc0.copy())
        torch_reference.write_kv(tk, tv, torch.from_numpy(k[valid]), torch.from_numpy(v[valid]),
                                 torch.from_numpy(slots[valid]))  # fmt: skip
        assert tk.numpy().tobytes() == kc.tobytes()
        assert tv.numpy().tobytes() == vc.tobytes()


def test_golden_fixtures_reproduce():
    """Committed fixtures (tests/golden/, made by tests/golden/make_golden.py from the fp64
    C oracle) still come out of both restatements."""
    from tests.golden.make_golden import load_fixtures

    for name, fx in load_fixtures().items():
        args = (fx["q"], fx["k_cache"], fx["v_cache"], fx["block_tables"], fx["seq_lens"], fx["query_start_loc"])
        out_c = oracle.paged_attention_f64(*args, float(fx["scale"]))
        np.testing.assert_allclose(out_c, fx["out"], atol=1e-12, err_msg=name)
        out_t = torch_attn(*args, float(fx["scale"]))
        np.testing.assert_allclose(out_t, fx["out"], atol=1e-10, err_msg=name)
