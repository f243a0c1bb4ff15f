#!/usr/bin/env python3
"""Benchmark of the HIP paged-attention backend on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-secondary]
    python bench.py --only N [--fp8]      # one BASELINE config (E4M3 KV caches with --fp8)
    python bench.py --sweep               # the reference's decode-kernel grid (bench/bench_kernel.py)
    python bench.py --probes              # attainable HBM read / copy and bf16 MFMA rates of this GPU

Headline workload: BASELINE config 2 (Llama-3.1-8B decode layer: 64 sequences, 32 q / 8 kv
heads, head_dim 128, block 16, contexts U[1024, 8192], bf16), the config the metric is
quoted on. One step = the backend's two calls of Attention.attend (src/kvserve/model.py:
106-108): write_kv (reshape_and_cache of the 64 new K/V rows) + forward (paged attention).
Inputs are resident in HBM; K timed steps run back to back between two synchronisations.

`value` is algorithmic GB/s of the step: unique K/V bytes read + Q read + O written +
block-table/length metadata + the cache write's read and write. The 1.2 GB working set is
~5x the 256 MB Infinity Cache, so back-to-back steps are HBM-cold.

Also printed in the same JSON line:
  roofline     - the decode kernel's algorithmic bytes / its mean launch duration, from HIP
                 events the library records around each of its kernels (kvh_profile_arm), vs
                 the 8 TB/s HBM peak; `traffic` is the kernel's HBM bytes per launch from two
                 child rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) calibrated on a plain
                 copy of known size;
  roofline_prefill - the same for C3's prefill kernel against the dense bf16 MFMA peak, its
                 `traffic` from the same two passes over a C3 child;
  cpu_baseline - the torch restatement of the reference's TorchAttention.forward (fp32, the
                 host's cores) on a bounded sample of the same workload;
  secondary    - the other BASELINE configs (C1, C3 prefill TFLOP/s + decode GB/s, C4 on
                 unique bytes, C5), and C2-C5 over E4M3 caches, timed the same way with
                 fewer steps;
  metadata_prep - per-step input preparation at C2 and C3: the reference's host path vs
                 block tables resident on the device (kvh_prepare_metadata);
  engine_decode_tok_s - Llama-3.2-1B / Llama-3.1-8B decode tokens/s of the engine harness
                 (kvserve_amd.engine, synthetic weights of the real shapes, HIP-graph decode),
                 next to the reference's RTX 4090 numbers.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
FLUSH_BYTES = 1 << 30  # written before each HBM-cold timed call
METRIC = "paged-attn decode HBM GB/s (% peak) + prefill TFLOP/s; 1B/8B decode tok/s"


class HipEvents:
    """hipEvent_t handles from the HIP runtime torch already loaded (same soname)."""

    def __init__(self, n: int):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            h = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(h)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.ev.append(h.value)
        self.array = (ctypes.c_void_p * n)(*self.ev)

    def elapsed_ms(self, a: int, b: int) -> float:
        self.hip.hipEventSynchronize(self.ev[b])
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[a], self.ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def close(self) -> None:
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def write_bytes(w, elem: int) -> int:
    """reshape_and_cache: each new K/V row read once and written once."""
    return 2 * 2 * w.num_tokens * w.num_kv_heads * w.head_dim * elem


def to_fp8_caches(b) -> dict:
    """Replace the batch's bf16 caches by E4M3 caches of the same values (scales 1 / 0.5),
    quantized on the device in slices; returns the scale arguments of the fp8 calls."""
    import torch

    kw = {"k_scale": 1.0, "v_scale": 0.5}
    for name in ("k_cache", "v_cache"):
        c, s = getattr(b, name), kw["k_scale" if name == "k_cache" else "v_scale"]
        c8 = torch.empty(c.shape, dtype=torch.float8_e4m3fn, device=c.device)
        step_blocks = max(1, (1 << 26) // c[0].numel())
        for b0 in range(0, c.shape[0], step_blocks):
            c8[b0 : b0 + step_blocks] = (c[b0 : b0 + step_blocks].float() / s).clamp(-448, 448).to(c8.dtype)
        setattr(b, name, c8)
        del c
    return kw


def measure(idx: int, steps: int, warmup: int, prof_iters: int, seed: int = 0, fp8: bool = False) -> dict:
    """One BASELINE config, bf16 q/out; fp8: the caches in E4M3 (scales 1 / 0.5, quantized
    from the same N(0, 1) values), K/V bytes counted at one byte per element."""
    import torch

    from kvserve_amd import HipAttention, _lib, last_launch_kernels, workloads

    w = workloads.baseline_config(idx, seed=seed)
    b = workloads.materialize(w, torch.bfloat16, "cuda:0", seed=seed)
    elem = 2
    kv_elem = 1 if fp8 else 2
    kw = to_fp8_caches(b) if fp8 else {}

    def step():
        HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping, **kw)
        return HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale, **kw)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / steps

    # the same step replayed from a HIP graph (as a serving engine's decode runs it): the GPU
    # time of the step without the host's per-call launch path
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        step()
    graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms_step_graph = start.elapsed_time(end) / steps
    del graph

    # HBM-cold timings: a 1 GiB read before each timed call evicts the 256 MB Infinity Cache
    # and the L2s (the reference flushes 256 MB for a 72 MB L2, bench/bench_kernel.py:36). A
    # read, not a write: written lines would stay dirty in the caches and their write-back
    # would be charged to the timed kernel.
    flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda:0")
    torch.cuda.synchronize()
    cold = []
    for _ in range(max(5, min(steps, 20))):
        flush.amax()
        start.record()
        step()
        end.record()
        end.synchronize()
        cold.append(start.elapsed_time(end))
    ms_step_cold = statistics.median(cold)

    # per-kernel durations from events the library records around each launch, each call
    # after a flush
    lib = _lib.load()
    ev = HipEvents(5)
    per_kernel: dict[str, list[float]] = {}
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping, **kw)
    for _ in range(prof_iters):
        flush.amax()
        lib.kvh_profile_arm(ev.array, 5)
        HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale, **kw)
        kinds = last_launch_kernels()
        for k, kind in enumerate(kinds[:4]):
            per_kernel.setdefault(kind, []).append(ev.elapsed_ms(k, k + 1))
    ev.close()
    del flush
    kernel_ms = {k: statistics.median(v) for k, v in per_kernel.items()}

    attn_bytes = w.algorithmic_bytes(elem, unique=True, kv_elem_bytes=kv_elem)
    # the cache write reads 16-bit rows and writes kv_elem-byte rows
    step_bytes = attn_bytes + write_bytes(w, elem) * (elem + kv_elem) // (2 * elem)
    res = {
        "workload": w.name + ("_fp8kv" if fp8 else ""),
        "ms_per_step": ms_step,
        "step_gbs": step_bytes / (ms_step * 1e-3) / 1e9,
        "ms_per_step_cold": ms_step_cold,
        "step_gbs_cold": step_bytes / (ms_step_cold * 1e-3) / 1e9,
        "ms_per_step_graph": ms_step_graph,
        "attn_bytes": attn_bytes,
        "kernel_ms": kernel_ms,
        "kernels": kinds,
    }
    if idx == 3:
        # prefill part: FLOPs of the 4 prefill sequences on the prefill kernel's own time;
        # decode part: bytes of the 512 decode sequences on the decode kernel's time
        pre = workloads.Workload("pre", w.query_lens[512:], w.seq_lens[512:], w.tables[512:], w.num_blocks,
                                 w.num_heads, w.num_kv_heads, w.head_dim, w.block_size)  # fmt: skip
        dec = workloads.Workload("dec", w.query_lens[:512], w.seq_lens[:512], w.tables[:512], w.num_blocks,
                                 w.num_heads, w.num_kv_heads, w.head_dim, w.block_size)  # fmt: skip
        if "prefill" in kernel_ms:
            res["prefill_tflops"] = pre.flops() / (kernel_ms["prefill"] * 1e-3) / 1e12
            res["prefill_frac_mfma"] = res["prefill_tflops"] / BF16_PEAK_TFLOPS
        res["decode_kernel_gbs"] = dec.algorithmic_bytes(elem, kv_elem_bytes=kv_elem) / (kernel_ms["decode"] * 1e-3) / 1e9
        res["prefill_gflop"] = pre.flops() / 1e9
    else:
        res["decode_kernel_gbs"] = attn_bytes / (kernel_ms["decode"] * 1e-3) / 1e9
        res["attn_gbs"] = attn_bytes / (sum(kernel_ms.values()) * 1e-3) / 1e9
    if idx == 4:
        res["logical_gbs"] = (w.algorithmic_bytes(elem, unique=False, kv_elem_bytes=kv_elem)
                              / (sum(kernel_ms.values()) * 1e-3) / 1e9)  # fmt: skip
    if idx == 5:
        res["tflops"] = w.flops() / (sum(kernel_ms.values()) * 1e-3) / 1e12
    del b
    torch.cuda.empty_cache()
    return res


# The reference's kernel sweep (bench/bench_kernel.py:58-82): 32 q / 8 kv heads, head_dim 64,
# block 16, bf16, one query per sequence over ctx - 1 cached tokens, batch x ctx with
# batch * ctx <= 64 * 8192; bytes = 2 B ctx Hkv D 2 (:81). Its published RTX 4090 figures
# (results/rtx4090/kernel_decode_attention.jsonl:1-14, 1008 GB/s peak) sit beside each point.
SWEEP_RTX4090_GBS = {
    (1, 512): 34.1, (1, 2048): 39.0, (1, 8192): 40.7, (8, 512): 234.1, (8, 2048): 292.6, (8, 8192): 308.5,
    (32, 512): 555.4, (32, 2048): 645.7, (32, 8192): 827.0, (64, 512): 619.0, (64, 2048): 773.7,
    (64, 8192): 900.1, (128, 512): 636.3, (128, 2048): 847.0,
}  # fmt: skip


def measure_sweep(iters: int = 50, warmup: int = 5) -> list[dict]:
    """The reference's decode-kernel grid on this GPU: the forward call (every kernel it launches)
    timed with events around it, each call after a 1 GiB read that evicts the caches (the
    reference flushes 256 MB for a 72 MB L2), median of `iters`; GB/s on the reference's byte
    formula and as a fraction of 8 TB/s. One JSON line per point."""
    import torch

    from kvserve_amd import HipAttention, _lib, last_launch_kernels, workloads

    H, Hkv, D, BS = 32, 8, 64, 16
    flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda:0")
    lib = _lib.load()
    ev = HipEvents(5)
    rows = []
    for batch in (1, 8, 32, 64, 128):
        for ctx in (512, 2048, 8192):
            if batch * ctx > 64 * 8192:
                continue
            w = workloads.custom(f"sweep_b{batch}_c{ctx}", [1] * batch, [ctx - 1] * batch, H, Hkv, D, BS, seed=0)
            b = workloads.materialize(w, torch.bfloat16, "cuda:0", seed=0)
            HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping)
            out = torch.empty_like(b.q)

            def fwd():
                return HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale, out=out)

            for _ in range(warmup):
                fwd()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            times, kern = [], []
            for _ in range(iters):
                flush.amax()
                lib.kvh_profile_arm(ev.array, 5)
                start.record()
                fwd()
                end.record()
                end.synchronize()
                times.append(start.elapsed_time(end))
                kinds = last_launch_kernels()
                kern.append(ev.elapsed_ms(0, len(kinds[:4])))
            ms = statistics.median(times)
            kms = statistics.median(kern)
            kv_bytes = 2 * batch * ctx * Hkv * D * 2
            gbs = kv_bytes / (ms * 1e-3) / 1e9
            ref = SWEEP_RTX4090_GBS.get((batch, ctx))
            row = {
                "batch": batch, "ctx": ctx, "ms": ms, "gbs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
                "kernels": kinds, "kernels_ms": kms, "kernels_gbs": kv_bytes / (kms * 1e-3) / 1e9,
                "rtx4090_gbs": ref, "rtx4090_frac": None if ref is None else ref / 1008.0,
            }  # fmt: skip
            print(json.dumps(row), flush=True)
            rows.append(row)
            del b, out
            torch.cuda.empty_cache()
    ev.close()
    return rows


def measure_probes(reps: int = 10) -> dict:
    """Attainable ceilings of this GPU from libkvhip's probes (kvh_probe): the HBM read rate of a
    streaming kernel with the decode kernels' 16-byte loads (4 GiB, 16x the Infinity Cache;
    ordinary and non-temporal loads), of a gather of scattered 4 KB pages (the decode kernels'
    access pattern, non-temporal), a copy's read + write rate (2 GiB each way), a copy of the C3 cache write's size (8.4 MB each
    way, after a 1 GiB read flush: the latency floor of a write that small), the dense bf16
    MFMA rate of the prefill kernel's instruction with 1 and 2 waves per SIMD, how an MFMA wave
    and a softmax-like VALU wave share a SIMD (each alone, then together), and what independent
    FMAs interleaved between one wave's own MFMAs add to its time. Medians of `reps` event-timed
    launches."""
    import torch

    from kvserve_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device=dev)

    def timed(kind, src, dst, nbytes, blocks, iters=0, cold=False):
        for _ in range(2):
            _lib.check(lib.kvh_probe(kind, src, dst, nbytes, blocks, iters, stream), "kvh_probe")
        ts = []
        for _ in range(reps):
            if cold:
                flush.amax()
            start.record()
            _lib.check(lib.kvh_probe(kind, src, dst, nbytes, blocks, iters, stream), "kvh_probe")
            end.record()
            end.synchronize()
            ts.append(start.elapsed_time(end))
        return statistics.median(ts)

    res = {"cus": cus}
    big = torch.randint(0, 1 << 30, ((4 << 30) // 4,), dtype=torch.int32, device=dev)
    for wgs_per_cu in (2, 4, 8):
        blocks = cus * wgs_per_cu
        sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
        ms = timed(0, big.data_ptr(), sink.data_ptr(), 4 << 30, blocks)
        res[f"stream_read_gbs_{wgs_per_cu}wg_per_cu"] = (4 << 30) / (ms * 1e-3) / 1e9
        # the same with non-temporal loads (the decode kernels' K/V loads)
        ms = timed(5, big.data_ptr(), sink.data_ptr(), 4 << 30, blocks)
        res[f"stream_read_nt_gbs_{wgs_per_cu}wg_per_cu"] = (4 << 30) / (ms * 1e-3) / 1e9
        ms = timed(6, big.data_ptr(), sink.data_ptr(), 4 << 30, blocks)
        res[f"page_gather_nt_gbs_{wgs_per_cu}wg_per_cu"] = (4 << 30) / (ms * 1e-3) / 1e9
    half = (2 << 30) // 4
    src, dst = big[:half], big[half:]
    ms = timed(1, src.data_ptr(), dst.data_ptr(), 2 << 30, cus * 8)
    res["copy_gbs_rw"] = 2 * (2 << 30) / (ms * 1e-3) / 1e9
    small = 2048 * 8 * 128 * 2 * 2  # the C3 cache write: 2048 tokens of K and V rows
    # one pass per thread: 8 loads in flight, then their 8 stores
    ms = timed(1, src.data_ptr(), dst.data_ptr(), small, small // 16 // (256 * 8), cold=True)
    res["copy_c3_write_size_us"] = ms * 1e3
    res["copy_c3_write_size_gbs_rw"] = 2 * small / (ms * 1e-3) / 1e9
    del big, src, dst
    iters = 20000
    for waves_per_simd in (1, 2):
        blocks = cus * waves_per_simd
        sink = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
        ms = timed(2, None, sink.data_ptr(), 0, blocks, iters)
        flop = blocks * 4 * 4 * iters * 16384
        res[f"mfma_bf16_tflops_{waves_per_simd}wave_per_simd"] = flop / (ms * 1e-3) / 1e12
    # co-issue: an MFMA wave and a VALU wave per SIMD, alone and together (VALU steps sized to
    # about the MFMA waves' time, the prefill chunk loop's balance)
    sink = torch.empty(cus * 512, dtype=torch.float32, device=dev)
    it_m, it_v = 4000, 1600
    co = {
        "mfma_alone_ms": timed(3, None, sink.data_ptr(), 0, cus, it_m),
        "valu_alone_ms": timed(3, None, sink.data_ptr(), it_v, cus, 0),
        "together_ms": timed(3, None, sink.data_ptr(), it_v, cus, it_m),
    }
    co["together_over_longer"] = co["together_ms"] / max(co["mfma_alone_ms"], co["valu_alone_ms"])
    res["coissue"] = co
    # one wave interleaving its own independent FMAs between MFMAs: time over MFMAs alone
    sink = torch.empty(cus * 2 * 256, dtype=torch.float32, device=dev)
    alone = timed(4, None, sink.data_ptr(), 0, cus * 2, 2000)
    res["interleave_over_mfma_alone"] = {
        f"{nv}_fma_per_mfma": timed(4, None, sink.data_ptr(), nv, cus * 2, 2000) / alone for nv in (1, 2, 4)
    }
    res["hbm_peak_gbs"] = HBM_PEAK_GBS
    res["bf16_peak_tflops"] = BF16_PEAK_TFLOPS
    del flush
    torch.cuda.empty_cache()
    return res


def cpu_baseline(idx: int, budget_s: float, seed: int = 0) -> dict:
    """The reference's torch attention (restated in oracle/torch_reference.py) in fp32 on the
    host cores, one sequence at a time, on the same bf16 values."""
    import torch

    from kvserve_amd import workloads
    from oracle import torch_reference

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    w = workloads.baseline_config(idx, seed=seed)
    b = workloads.materialize(w, torch.bfloat16, "cuda:0", seed=seed)
    # stage the sample on the host once: the timed region is the CPU attention only
    seqs = []
    for s in range(len(w.seq_lens)):
        table = torch.tensor(w.tables[s], device="cuda:0")
        q0 = sum(w.query_lens[:s])
        seqs.append((
            b.q[q0 : q0 + w.query_lens[s]].float().cpu(),
            b.k_cache.index_select(0, table).float().cpu(),
            b.v_cache.index_select(0, table).float().cpu(),
            torch.arange(len(w.tables[s]), dtype=torch.long)[None],
            torch.tensor([w.seq_lens[s]]),
            torch.tensor([w.query_lens[s]]),
            workloads.Workload("s", [w.query_lens[s]], [w.seq_lens[s]], [w.tables[s]], w.num_blocks, w.num_heads,
                               w.num_kv_heads, w.head_dim, w.block_size).algorithmic_bytes(2),
        ))  # fmt: skip
    torch_reference.forward(*seqs[0][:6], w.scale)  # warm-up, untimed
    done_bytes, spent, n, passes = 0, 0.0, 0, 0
    while spent < budget_s and passes < 50:
        passes += 1
        for q, kc, vc, bt, sl, ql, nbytes in seqs:
            t0 = time.perf_counter()
            torch_reference.forward(q, kc, vc, bt, sl, ql, w.scale)
            spent += time.perf_counter() - t0
            done_bytes += nbytes
            n += 1
    del b
    torch.cuda.empty_cache()
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": done_bytes / spent / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{passes} pass(es) over the {len(w.seq_lens)} sequences of {w.name} ({n} calls, one sequence "
        f"per call), fp32 torch gather+repeat_interleave+masked SDPA, {spent:.1f} s timed",
        "cpu_model": cpu,
        "ms_per_seq": 1e3 * spent / max(n, 1),
    }


# The reference's published engine decode rates (RTX 4090, graph mode, 512-token prompts):
# results/rtx4090/decode_graphs.jsonl:1-5 for Llama-3.2-1B; README.md:279 for Llama-3.1-8B.
REF_DECODE_TOK_S = {"llama_3_2_1b": {1: 253, 8: 1725, 32: 5872, 64: 9588, 128: 14526},
                    "llama_3_1_8b": {1: 57, 8: 399, 32: 1427}}  # fmt: skip


def measure_engine(name: str, batches: list[int], prompt_len: int = 512, steps: int = 50, seed: int = 0) -> dict:
    """Decode tokens/s of the engine harness with synthetic weights of the model's real shape
    (bench/bench_decode.py:22-39 of the reference): prefill `batch` prompts of prompt_len
    tokens, 3 warm-up decode steps, then `steps` timed decode steps replayed from HIP graphs,
    each step = host metadata + graph replay + logits + greedy argmax read back to the host."""
    import torch

    from kvserve_amd import HipAttention
    from kvserve_amd.engine import LLAMA_3_1_8B, LLAMA_3_2_1B
    from kvserve_amd.engine.model import build_model
    from kvserve_amd.engine.runner import ModelRunner, Sequence

    cfg = {"llama_3_2_1b": LLAMA_3_2_1B, "llama_3_1_8b": LLAMA_3_1_8B}[name]
    max_len = prompt_len + steps + 16
    model = build_model(cfg, "cuda:0", torch.bfloat16, max_len, backend=HipAttention, seed=seed)
    blocks = max(batches) * -(-max_len // 16) + 16
    runner = ModelRunner(model, num_blocks=blocks, block_size=16, max_model_len=max_len, decode_graphs=True,
                         piecewise_graphs=False, max_graph_batch=max(batches))  # fmt: skip
    out = {}
    for b in batches:
        seqs = [Sequence([1000 + (i * 7 + j) % 30000 for j in range(prompt_len)]) for i in range(b)]
        runner.prefill(seqs)
        for _ in range(3):
            runner.decode(seqs)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            runner.decode(seqs)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / steps * 1e3
        ref = REF_DECODE_TOK_S[name].get(b)
        out[str(b)] = {"ms_per_step": ms, "tok_s": b / ms * 1e3, "rtx4090_tok_s": ref,
                       "vs_rtx4090": (b / ms * 1e3) / ref if ref else None}  # fmt: skip
        for sq in seqs:
            runner.release(sq)
    del runner, model
    torch.cuda.empty_cache()
    return {"prompt_len": prompt_len, "steps": steps, "weights": "synthetic N(0, 0.02), real shapes", "batches": out}


def measure_metadata(idx: int, steps: int = 30) -> dict:
    """Per-step input preparation: the reference's host path (slots per sequence,
    build_metadata, token and position tensors; model_runner.py:114-125, 165-197) against
    DeviceMetadata (resident block tables, one packed upload, kvh_prepare_metadata), each
    step ended by a synchronisation. Every step advances each sequence by its query length
    (decode: one token; C3's prefill chunks: 384), appending blocks to its table as the
    reference's allocator would, so the resident tables receive only the new entries."""
    import torch

    from kvserve_amd import workloads
    from kvserve_amd.attention import build_metadata
    from kvserve_amd.metadata import DeviceMetadata

    w = workloads.baseline_config(idx)
    bs, dev = w.block_size, torch.device("cuda:0")
    B = len(w.query_lens)
    seqs = [list(t) for t in w.tables]
    qlens = list(w.query_lens)
    growth = [(steps + 2) * q // bs + 2 for q in qlens]
    spare = iter(())
    starts = [s - q for s, q in zip(w.seq_lens, w.query_lens)]
    ids = [(7 * i) % 128000 for i in range(sum(qlens))]
    width = max(len(t) + g for t, g in zip(seqs, growth))
    dm = DeviceMetadata(dev, B, width, bs, sum(qlens))

    def advance():
        for b in range(B):
            starts[b] += qlens[b]
            while starts[b] + qlens[b] > len(seqs[b]) * bs:
                seqs[b].append(next(spare))

    def host_step():
        slots, pos, seq_lens = [], [], []
        for t, st, q in zip(seqs, starts, qlens):
            slots += workloads.slots_for(t, bs, st, q)
            pos += range(st, st + q)
            seq_lens.append(st + q)
        build_metadata(dev, seqs, slots, seq_lens, qlens)
        torch.tensor(ids, device=dev), torch.tensor(pos, device=dev)
        torch.cuda.synchronize()

    def device_step():
        dm.build([(b, seqs[b]) for b in range(B)], starts, qlens, ids)
        torch.cuda.synchronize()

    out = {"workload": w.name, "batch": B, "tokens": sum(qlens), "max_table": max(len(t) for t in seqs)}
    saved = (list(starts), [list(t) for t in seqs])
    for name, fn in (("host_reference_ms", host_step), ("device_ms", device_step)):
        starts[:], seqs[:] = list(saved[0]), [list(t) for t in saved[1]]
        spare = iter(range(w.num_blocks, w.num_blocks + sum(growth)))
        fn()  # first step: the device path uploads every table
        advance()
        times = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fn()
            times.append((time.perf_counter() - t0) * 1e3)
            advance()
        out[name] = statistics.median(times)
    out["speedup"] = out["host_reference_ms"] / out["device_ms"]
    return out


CALIB_ELEMS = 1 << 27  # bf16 elements of the calibration copy: 256 MiB read + 256 MiB written


def pmc_child(idx: int = 2, fp8: bool = False) -> None:
    """Workload of one counter pass: a plain copy of known size (torch.neg on bf16: reads and
    writes CALIB bytes, a kernel whose name holds "neg_kernel"), then one BASELINE config's
    write + three forwards (C2 unless told otherwise; E4M3 caches with fp8), each forward after a
    1 GiB read that evicts the caches, as the HBM-cold timings are taken."""
    import torch

    from kvserve_amd import HipAttention, workloads

    x = torch.ones(CALIB_ELEMS, dtype=torch.bfloat16, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(2):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    del x, y
    w = workloads.baseline_config(idx)
    b = workloads.materialize(w, torch.bfloat16, "cuda:0")
    kw = to_fp8_caches(b) if fp8 else {}
    flush = torch.zeros(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda:0")
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping, **kw)
    for _ in range(3):
        flush.amax()
        HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale, **kw)
    torch.cuda.synchronize()


def measure_traffic(timeout_s: int = 150, idx: int = 2, kernel: str = "pa_decode_kernel") -> dict | None:
    """HBM bytes per launch of `kernel` in BASELINE config `idx` from two rocprofv3 --pmc passes
    (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the same counter reads
    for the calibration copy of known size. None when rocprofv3 is missing or a pass fails."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not Path(prof).exists():
        return None
    calib_bytes = CALIB_ELEMS * 2
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="kvh_pmc_", dir="/tmp")
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
               sys.executable, str(ROOT / "bench.py"), "--pmc-child", "--only", str(idx)]  # fmt: skip
        env = dict(os.environ, TMPDIR="/tmp")
        try:
            subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, check=True,
                           stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)  # fmt: skip
        except (subprocess.SubprocessError, OSError):
            shutil.rmtree(d, ignore_errors=True)
            return None
        calib, dec = [], []
        for f in Path(d).rglob("*counter_collection.csv"):
            for row in csv.DictReader(open(f)):
                if row.get("Counter_Name") != counter:
                    continue
                name, val = row["Kernel_Name"], float(row["Counter_Value"]) * 1024.0
                if "neg_kernel" in name:
                    calib.append(val)
                elif kernel in name:
                    dec.append(val)
        shutil.rmtree(d, ignore_errors=True)
        if not calib or not dec:
            return None
        factor = statistics.mean(calib) / calib_bytes
        out[counter] = {"raw_bytes": statistics.mean(dec), "calib_factor": factor,
                        "bytes": statistics.mean(dec) / factor}  # fmt: skip
    return out


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--prof-iters", type=int, default=20)
    p.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--only", type=int, default=0, help="run just this config (1-5) and print its record")
    p.add_argument("--fp8", action="store_true", help="with --only: E4M3 KV caches")
    p.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc passes")
    p.add_argument("--no-engine", action="store_true", help="skip the 1B/8B engine decode tokens/s")
    p.add_argument("--engine-only", action="store_true", help="run just the engine decode tokens/s")
    p.add_argument("--probes", action="store_true",
                   help="attainable HBM read / copy and bf16 MFMA rates of this GPU (libkvhip's probes)")
    p.add_argument("--sweep", action="store_true",
                   help="the reference's decode-kernel grid (32/8 heads, D 64, batch x ctx) beside its RTX 4090 GB/s")
    p.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    args = p.parse_args()
    if args.pmc_child:
        pmc_child(args.only or 2, args.fp8)
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one GPU only: this build targets a single MI355X (its kernels run on one "
            "GPU's share of the work; the multi-GPU sharding is a design note, not a run). Use --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from kvserve_amd import hip_available

    if not hip_available():
        print("bench.py needs a ROCm GPU and kvserve_amd/lib/libkvhip.so (python -m kvserve_amd.build)", file=sys.stderr)
        return 1

    if args.only:
        print(json.dumps(measure(args.only, args.steps, args.warmup, args.prof_iters, fp8=args.fp8)), flush=True)
        return 0
    if args.sweep:
        measure_sweep()
        return 0
    if args.probes:
        print(json.dumps(measure_probes()), flush=True)
        return 0
    engine_batches = {"llama_3_2_1b": [1, 8, 32, 64, 128], "llama_3_1_8b": [1, 8, 32, 64]}
    if args.engine_only:
        for name, bs in engine_batches.items():
            print(json.dumps({name: measure_engine(name, bs)}), flush=True)
        return 0

    head = measure(2, args.steps, args.warmup, args.prof_iters)
    print(f"# c2: {head['ms_per_step']:.4f} ms/step, kernels {head['kernel_ms']}", file=sys.stderr, flush=True)
    dec_ms = head["kernel_ms"]["decode"]
    achieved = head["attn_bytes"] / (dec_ms * 1e-3) / 1e9
    record = {
        "metric": METRIC,
        "value": head["step_gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/K/V, shuffled 40k-block pool)",
        "config": {
            "workload": "c2_8b_decode: BASELINE config 2, Llama-3.1-8B layer decode",
            "batch": 64,
            "num_heads": 32,
            "num_kv_heads": 8,
            "head_dim": 128,
            "block_size": 16,
            "context": "U[1024,8192]",
            "step": "write_kv + forward",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
            "kernel": "pa_decode_kernel<BF16,128,1> (stream-K decode)",
            "kernel_ms": dec_ms,
        },
        "kernel_ms": head["kernel_ms"],
    }
    if not args.no_traffic:
        t = measure_traffic()
        if t is not None:
            rl = record["roofline"]
            rl["traffic"] = t["FETCH_SIZE"]["bytes"] + t["WRITE_SIZE"]["bytes"]
            rl["traffic_detail"] = {
                "fetch_bytes": t["FETCH_SIZE"]["bytes"],
                "write_bytes": t["WRITE_SIZE"]["bytes"],
                "fetch_calib_factor": t["FETCH_SIZE"]["calib_factor"],
                "write_calib_factor": t["WRITE_SIZE"]["calib_factor"],
                "algorithmic_bytes": head["attn_bytes"],
            }
        print(f"# traffic: {t}", file=sys.stderr, flush=True)
    if not args.no_secondary:
        sec = {}
        runs = [(idx, False) for idx in (1, 3, 4, 5)] + [(idx, True) for idx in (2, 3, 4, 5)]
        for idx, kv8 in runs:
            r = measure(idx, max(20, args.steps), 3, max(10, args.prof_iters), fp8=kv8)
            print(f"# c{idx}{' fp8 kv' if kv8 else ''}: {r}", file=sys.stderr, flush=True)
            sec[r["workload"]] = {k: v for k, v in r.items() if k not in ("workload", "attn_bytes")}
        record["secondary"] = sec
        c3 = sec.get("c3_mixed_prefill", {})
        if "prefill_tflops" in c3:
            record["roofline_prefill"] = {
                "bound": "mfma",
                "achieved": c3["prefill_tflops"],
                "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": c3["prefill_tflops"] / BF16_PEAK_TFLOPS,
                "traffic": None,
                "kernel": "pa_prefill_kernel<BF16,128,false> (stream-K prefill tiles)",
                "kernel_ms": c3["kernel_ms"]["prefill"],
                "workload": "c3_mixed_prefill: the 4 prefill chunks of 384 tokens (HBM-cold, median)",
                "gflop": c3["prefill_gflop"],
            }
            if not args.no_traffic:
                # what the prefill kernel moves: Q, the K/V chunks of its tiles (re-read by the
                # units that split a tile), its output rows and the split tiles' fp32 partials
                t = measure_traffic(idx=3, kernel="pa_prefill_kernel")
                if t is not None:
                    rp = record["roofline_prefill"]
                    rp["traffic"] = t["FETCH_SIZE"]["bytes"] + t["WRITE_SIZE"]["bytes"]
                    rp["traffic_detail"] = {"fetch_bytes": t["FETCH_SIZE"]["bytes"], "write_bytes": t["WRITE_SIZE"]["bytes"]}
                print(f"# prefill traffic: {t}", file=sys.stderr, flush=True)
    if not args.no_secondary:
        meta = {}
        for idx in (2, 3):
            m = measure_metadata(idx)
            print(f"# metadata c{idx}: {m}", file=sys.stderr, flush=True)
            meta[m.pop("workload")] = m
        record["metadata_prep"] = meta
    if not args.no_engine:
        eng = {}
        for name, bs in engine_batches.items():
            eng[name] = measure_engine(name, bs)
            print(f"# engine {name}: {eng[name]}", file=sys.stderr, flush=True)
        record["engine_decode_tok_s"] = eng
    if not args.no_cpu:
        record["cpu_baseline"] = cpu_baseline(2, args.cpu_budget)
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
