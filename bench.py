"""Benchmark of the gfx950 attention path on BASELINE.json's configurations.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|cfg1|cfg2|cfg3|cfg4|cfg5|proj]
                    [--no-cpu] [--calibrate]

Prints ONE JSON line. `value` is BASELINE's headline metric on its headline
workload: achieved HBM GB/s of Llama-3-8B-shaped paged Q8_0 decode attention
at batch 64 (config 3), with every input resident in HBM. The other
configurations are reported under "secondary": config 1 (SmolLM decode
latency, eagerly and with its layers' calls replayed as one HIP graph),
config 2 (32 layers of f32 decode), config 4 (4x2048 causal prefill,
TFLOP/s, fp32 and bf16-input), config 5 (Gemma-2 windowed + global decode)
and "proj", the Q8_0 QKV projection matvec beside attention (1 and 64 tokens).

Timing. A step is one gla_decode (or gla_prefill, or gla_matvec_q8_0) call
over the whole batch for one layer. W untimed steps, then K steps (at least
20), each between its own pair of HIP events recorded on the library's stream
(the stream the kernels run on), with a device synchronisation on both sides
of the timed region. Every leg reports the median, min, max and mean of the
per-step times ("timing_us"); rates use the median. Consecutive steps
alternate between layers whose K/V live in different memory, so the 256 MB
Infinity Cache cannot serve repeats.

Settle. A leg's set-up (pool writes, uploads, host work) leaves the GPU
mostly idle for a while, and the first ~100 calls after such a gap run
through the power controller's transient: at cfg3 (K=50) the median was
108.4-109.0 us against 101.6-101.9 us in sustained work, bf16 prefill
185-192 us against 158-162 us. So right before each leg's W warmup steps the
bench runs a different kernel of the leg's kind -- ~0.1 s of streaming reads
of a 1 GiB buffer for the HBM-bound legs, ~0.3 s of the bf16 MFMA loop on
random operands for the prefill legs (glint_amd/csrc/gla_probe.hip) -- and
the timed steps measure what the path sustains. The W warmup and K timed steps are the leg's own, unchanged;
"settle" in the JSON says what ran. --no-settle leaves it out (to measure its effect,
profiles/settle_effect.md).

roofline: algorithmic bytes of one call (unique K/V bytes of the attended
positions, page-table entries, q and out) divided by the call's median
duration; the call is decode_q8_mfma_kernel + decode_q8_combine_kernel.
`traffic` comes from the rocprofv3 request-size counter summary committed in
profiles/decode_q8_cfg3_pmc.md (calibrated against a page-copy kernel of
known size, see --calibrate), or is null when that file is absent.

cpu_baseline: the C restatement of Glint's CPU flash path (oracle/), compiled
on this host with gcc -O3 -march=native -ffp-contract=off, on the same inputs,
on a bounded sample: one thread for configs 1 and 2 (Glint's single-sequence
decode is serial over heads, src/transformer/forward.rs:254-269), otherwise
parallel over sequences (forward.rs:1499-1502) or query positions
(forward.rs:927-931) on the cores this process may use (Rayon's default
width), fewer only if OMP_NUM_THREADS says so (a shared host's CPU share).
`cores` is the thread count; `host_cores` what the process
could see.

errors: the GPU output for the cpu_baseline sample (the same call, after the
timed region) against the oracle's: max_abs_err; max_rel_err over elements
with |want| >= 1e-3; frac_of_tolerance = max of err / max(abs_tol, rel_tol *
|want|) (<= 1 is within the bar: abs 1e-4 / rel 1e-3 for fp32, 3e-2 / 3e-2
for the bf16-input prefill).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import re
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from glint_amd import synth  # noqa: E402
from glint_amd.attn import GpuBackend  # noqa: E402

METRIC = "decode-attn HBM GB/s (% peak) + prefill TFLOP/s, Llama-3-8B GQA shape"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
PAGE = 16
SEED = 0x61F7
PMC_SUMMARY = ROOT / "profiles" / "decode_q8_cfg3_pmc.md"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent timing on a given stream, through the HIP runtime the library loaded."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so.7")
        self.h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipEventDestroy.argtypes = [C.c_void_p]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]

    def create(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def destroy(self, e) -> None:
        self.h.hipEventDestroy(e)

    def record(self, e, stream: int) -> None:
        assert self.h.hipEventRecord(e, C.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.h.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return float(ms.value)


class Timing:
    """Per-call durations (ms) of the samples of one timed region, and the region's total."""

    def __init__(self, per_ms: list[float], region_ms: float, group: int):
        self.per = np.asarray(per_ms, np.float64)
        self.region_ms = region_ms
        self.group = group

    @property
    def median_ms(self) -> float:
        return float(np.median(self.per))

    def summary_us(self) -> dict:
        us = self.per * 1e3
        return {"median": round(float(np.median(us)), 2), "min": round(float(us.min()), 2),
                "max": round(float(us.max()), 2), "mean": round(float(us.mean()), 2), "samples": int(us.size),
                "calls_per_sample": self.group,
                "region_mean": round(self.region_ms * 1e3 / (us.size * self.group), 2)}


def time_steps(be: GpuBackend, ev: HipEvents, step, samples: int, warmup: int, group: int = 1) -> Timing:
    """W untimed calls, then `samples` samples of `group` consecutive calls, each sample between
    its own event pair on the library's stream (device synchronisation on both sides of the
    timed region); per-call time of a sample = its duration / group. One call per sample for the
    ~0.1-1 ms steps; a group (one model step's layers) for the few-microsecond ones, where an
    event pair per call would cost as much as the call and leave the GPU waiting on the host."""
    for i in range(warmup):
        step(i)
    be.sync()
    pairs = [(ev.create(), ev.create()) for _ in range(samples)]
    n = warmup
    for a, b in pairs:
        ev.record(a, be.stream)
        for _ in range(group):
            step(n)
            n += 1
        ev.record(b, be.stream)
    be.sync()
    per = [ev.elapsed_ms(a, b) / group for a, b in pairs]
    region = ev.elapsed_ms(pairs[0][0], pairs[-1][1])
    for a, b in pairs:
        ev.destroy(a)
        ev.destroy(b)
    return Timing(per, region, group)


def error_figures(got, want, abs_tol: float, rel_tol: float) -> dict:
    """The GPU output of a sample against the oracle's (definitions in the module docstring)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    big = np.abs(want) >= 1e-3
    rel = float((err[big] / np.abs(want[big])).max()) if big.any() else 0.0
    bar = float((err / np.maximum(abs_tol, rel_tol * np.abs(want))).max())
    return {"max_abs_err": float(f"{err.max():.3g}"), "max_rel_err": float(f"{rel:.3g}"),
            "frac_of_tolerance": round(bar, 4), "tolerance": f"abs {abs_tol:g} / rel {rel_tol:g}",
            "elements": int(err.size)}


class CpuBaseline:
    """The oracle built for this host (oracle.build_native), its thread count and a host
    description; falls back to the prebuilt portable oracle when gcc fails."""

    def __init__(self):
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as orc
        self.orc = orc
        try:
            self.L = orc.build_native(Path(tempfile.mkdtemp(prefix="glint_oracle_")))
            self.build = "gcc " + " ".join(orc.NATIVE_FLAGS)
        except Exception as ex:  # noqa: BLE001 -- the portable build is the fallback
            self.L = orc.lib()
            self.build = f"prebuilt oracle/liboracle.so (-O2 -march=x86-64-v3; native build failed: {ex})"
        self.host_cores = orc.host_cores()
        self.threads = orc.threads()
        self.cpu = cpu_model()

    def describe(self, d: dict, threads: int) -> dict:
        d.update(cores=threads, host_cores=self.host_cores, cpu=self.cpu, build=self.build)
        return d


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def q8_token_bytes(n_kv: int, d: int) -> int:
    return 2 * n_kv * (d + (d // 32) * 2)  # K and V quants + f16 block scales


def unique_rows(pb: synth.PagedBatch) -> tuple[int, int]:
    """(unique physical rows read, logical rows read) by a decode over pb."""
    rows = []
    for b in range(len(pb.ctx)):
        pos = np.arange(pb.kv_start[b], pb.kv_start[b] + pb.kv_len[b])
        rows.append(pb.table[b, pos // PAGE].astype(np.int64) * PAGE + pos % PAGE)
    allr = np.concatenate(rows) if rows else np.zeros(0, np.int64)
    return int(len(np.unique(allr))), int(len(allr))


def pages_read(pb: synth.PagedBatch) -> int:
    n = 0
    for b in range(len(pb.ctx)):
        if pb.kv_len[b] > 0:
            n += (int(pb.kv_start[b] + pb.kv_len[b] - 1) // PAGE) - int(pb.kv_start[b]) // PAGE + 1
    return n


def write_pool_chunked(pool, seed_k, seed_v, first_page, n_pages, kv_dim, k_mul=1.0, keep_q8=False):
    """Generate N(0,1) rows page-chunk by page-chunk and write them (quantise-on-write);
    optionally keep the host Q8_0 bytes (Glint's 34-byte blocks) for the CPU baseline."""
    chunk = max(1, (1 << 16) // PAGE)
    kq = vq = None
    if keep_q8:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oracle as orc
        rb = orc.q8_row_bytes(kv_dim)
        kq = np.empty((n_pages * PAGE, rb), np.uint8)
        vq = np.empty_like(kq)
    for p0 in range(0, n_pages, chunk):
        n = min(chunk, n_pages - p0)
        rows, k, v = synth.pool_rows(seed_k, seed_v, first_page + p0, n, kv_dim, k_mul)
        pool.write_rows(rows, k, v)
        if keep_q8:
            kq[p0 * PAGE:(p0 + n) * PAGE] = orc.q8_quantize_rows(k)
            vq[p0 * PAGE:(p0 + n) * PAGE] = orc.q8_quantize_rows(v)
    return kq, vq


# --------------------------------------------------------------------------- decode workloads
class PagedDecode:
    """Configs 3 and 5: batched decode over a paged Q8_0 pool, one layer per entry of
    `windows` (None: global attention), all layers in one pool."""

    def __init__(self, be, name, H, Hkv, d, B, ctx_lo, ctx_hi, prefix, softcap, windows, k_mul, seed):
        self.be, self.name, self.H, self.Hkv, self.d = be, name, H, Hkv, d
        self.kv_dim = Hkv * d
        self.scale = float(1.0 / np.sqrt(d))
        self.softcap = softcap
        self.ctx = synth.uniform_int(seed, ctx_lo, ctx_hi, B)
        base = synth.paged_batch(seed + 1, self.ctx, prefix_tokens=prefix)
        self.n_layers = len(windows)
        self.layers = []
        self.pool = be.create_page_pool(base.n_pages * self.n_layers, Hkv, d, "q8")
        self.host_q8 = None
        tok = q8_token_bytes(Hkv, d)
        for li, w in enumerate(windows):
            pb = synth.windowed(base, w)
            table = pb.table + li * base.n_pages
            kq, vq = write_pool_chunked(self.pool, synth.tensor_seed(seed, 3, li, 1), synth.tensor_seed(seed, 3, li, 2),
                                        li * base.n_pages, base.n_pages, self.kv_dim, k_mul, keep_q8=(li == 0))
            if li == 0:
                self.host_q8 = (kq, vq, pb)
            q = synth.normal(synth.tensor_seed(seed, 3, li, 3), (B, H, d))
            uniq, logical = unique_rows(pb)
            self.layers.append(dict(
                pb=pb, q=be.buffer(q), q_host=q, out=be.empty(q.nbytes),
                start=be.buffer(pb.kv_start), len=be.buffer(pb.kv_len), table=be.buffer(table),
                start_host=np.ascontiguousarray(pb.kv_start, np.int32), len_host=np.ascontiguousarray(pb.kv_len, np.int32),
                stride=table.shape[1], max_len=int(pb.kv_len.max()),
                bytes=uniq * tok + pages_read(pb) * 4 + 2 * q.nbytes,
                bytes_logical=logical * tok + pages_read(pb) * 4 + 2 * q.nbytes,
                attended=int(pb.kv_len.sum()),
            ))
        be.sync()

    def step(self, i):
        L = self.layers[i % self.n_layers]
        # the engine keeps every sequence's position on the host and passes the
        # host copies along (they size the launch; see gla_decode_args)
        self.be.decode(self.pool, L["q"], L["out"], L["start"], L["len"], len(self.ctx), L["max_len"], self.H,
                       self.scale, self.softcap, page_table=L["table"], page_table_stride=L["stride"],
                       kv_start_host=L["start_host"], kv_len_host=L["len_host"])

    def bytes_per_step(self):
        return float(np.mean([L["bytes"] for L in self.layers]))

    def cpu_baseline(self, cb: CpuBaseline, min_seconds=10.0, max_reps=200):
        """Layer 0 of every sequence through the oracle's decode_batch, one task per sequence.
        Returns (baseline, the oracle's output [B][H][d])."""
        orc = cb.orc
        kq, vq, pb = self.host_q8
        pk = kq.reshape(-1, PAGE, kq.shape[-1])
        pv = vq.reshape(-1, PAGE, vq.shape[-1])
        stores = [orc.paged_q8(pk, pv, self.kv_dim, pb.table[b:b + 1], L=cb.L) for b in range(len(self.ctx))]
        L0 = self.layers[0]
        q = L0["q_host"].reshape(len(self.ctx), -1)
        nt = cb.threads
        reps, t0 = 0, time.perf_counter()
        while True:
            out = orc.decode_batch(q, stores, 0, pb.kv_start, pb.kv_len, self.H, self.Hkv, self.d, self.scale,
                                   self.softcap, n_threads=nt)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min_seconds or reps >= max_reps:
                break
        base = dict(value=round(L0["bytes"] * reps / el / 1e9, 3), unit="GB/s", kind="port",
                    sample=f"{reps} x layer 0 of {self.name} (all {len(self.ctx)} sequences, same inputs), "
                           f"{el:.1f} s; oracle decode_batch, one task per sequence")
        return cb.describe(base, nt), out.reshape(len(self.ctx), self.H, self.d)

    def gpu_sample(self):
        """The GPU output of layer 0 (the cpu_baseline sample)."""
        self.step(0)
        self.be.sync()
        return self.layers[0]["out"].download((len(self.ctx), self.H, self.d))

    def drop_device(self):
        """Free the device pool and buffers (the CPU leg reads host copies only)."""
        self.pool.destroy()
        for L in self.layers:
            for key in ("q", "out", "start", "len", "table"):
                L.pop(key).free()


class ContigDecode:
    """Configs 1 and 2: single-sequence f32 decode over contiguous caches, `n_layers`
    layers back to back with independent seeds (config 2: 32 layers = 1 GiB of K/V)."""

    def __init__(self, be, n_layers, ctx, H, Hkv, d, seed, name):
        self.be, self.H, self.Hkv, self.d, self.ctx, self.name = be, H, Hkv, d, ctx, name
        self.kv_dim = Hkv * d
        self.n_layers = n_layers
        self.scale = float(1.0 / np.sqrt(d))
        self.cache = be.create_kv_cache(n_layers, ctx, Hkv, d, "f32", 1)
        self.host = None
        for layer in range(n_layers):
            rows = np.array([self.cache.row_id(0, layer, 0)], np.int64) + np.arange(ctx)
            k = synth.normal_rows(synth.tensor_seed(seed, 2, layer, 1), ctx, self.kv_dim)
            v = synth.normal_rows(synth.tensor_seed(seed, 2, layer, 2), ctx, self.kv_dim)
            for i in range(0, ctx, 1 << 14):
                self.cache.write_rows(rows[i:i + (1 << 14)], k[i:i + (1 << 14)], v[i:i + (1 << 14)])
            if layer == 0:
                self.host = (k, v)
        self.q_host = [synth.normal(synth.tensor_seed(seed, 2, layer, 3), (1, H, d)) for layer in range(n_layers)]
        self.q = [be.buffer(x) for x in self.q_host]
        self.out = be.empty(H * d * 4)
        self.start = be.buffer(np.zeros(1, np.int32))
        self.len = be.buffer(np.full(1, ctx, np.int32))
        be.sync()

    def step(self, i):
        layer = i % self.n_layers
        self.be.decode(self.cache, self.q[layer], self.out, self.start, self.len, 1, self.ctx, self.H, self.scale,
                       layer=layer)

    def bytes_per_step(self):
        return float(2 * self.ctx * self.kv_dim * 4 + 2 * self.H * self.d * 4)

    def cpu_baseline(self, cb: CpuBaseline, min_seconds=3.0, max_reps=2000):
        """Layer 0 through attn_heads_cpu, one thread (Glint's single-sequence decode is serial
        over heads). Returns (baseline, the oracle's output [1][H][d])."""
        orc = cb.orc
        k, v = self.host
        st = orc.kv_cache(k[None], v[None], L=cb.L)
        q = self.q_host[0].reshape(-1)
        reps, t0 = 0, time.perf_counter()
        while True:
            out = orc.attn_heads_cpu(q, st, 0, 0, self.ctx, self.H, self.H // self.Hkv, self.d, self.scale)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min_seconds or reps >= max_reps:
                break
        base = dict(value=round(self.bytes_per_step() * reps / el / 1e9, 3), unit="GB/s", kind="port",
                    sample=f"{reps} x layer 0 of {self.name} (attn_heads_cpu, serial over heads as Glint), "
                           f"{el:.1f} s", us_per_layer=round(el / reps * 1e6, 2))
        return cb.describe(base, 1), out.reshape(1, self.H, self.d)

    def gpu_sample(self):
        self.step(0)
        self.be.sync()
        return self.out.download((1, self.H, self.d))

    def drop_device(self):
        self.cache.destroy()
        for buf in self.q + [self.out, self.start, self.len]:
            buf.free()
        self.q = []


class Prefill:
    """Config 4: causal prefill of 4 prompts x 2048 over an f32 KV cache (2 layers alternating)."""

    def __init__(self, be, B=4, S=2048, H=32, Hkv=8, d=128, seed=0x4444):
        self.be, self.B, self.S, self.H, self.Hkv, self.d = be, B, S, H, Hkv, d
        self.kv_dim = Hkv * d
        self.scale = float(1.0 / np.sqrt(d))
        self.n_layers = 2
        self.cache = be.create_kv_cache(self.n_layers, S, Hkv, d, "f32", B)
        self.host = None
        self.q = []
        for layer in range(self.n_layers):
            for b in range(B):
                rows = np.array([self.cache.row_id(b, layer, 0)], np.int64) + np.arange(S)
                k = synth.normal_rows(synth.tensor_seed(seed, 4, layer * 8 + b, 1), S, self.kv_dim)
                v = synth.normal_rows(synth.tensor_seed(seed, 4, layer * 8 + b, 2), S, self.kv_dim)
                self.cache.write_rows(rows, k, v)
                if layer == 0 and b == 0:
                    self.host = (k, v)
            qh = synth.normal(synth.tensor_seed(seed, 4, layer, 3), (B * S, H, d))
            if layer == 0:
                self.q0_host = qh
            self.q.append(be.buffer(qh))
        self.out = be.empty(B * S * H * d * 4)
        self.q_start = be.buffer(np.arange(B + 1, dtype=np.int32) * S)
        self.pos = be.buffer(np.zeros(B, np.int32))
        self.precision = "f32"
        be.sync()

    def step(self, i):
        layer = i % self.n_layers
        self.be.prefill(self.cache, self.q[layer], self.out, self.q_start, self.pos, self.B, self.S, self.H,
                        self.scale, layer=layer, precision=self.precision)

    def flops_per_step(self):
        return float(4 * self.B * self.H * self.d * self.S * (self.S + 1) // 2)

    def cpu_baseline(self, cb: CpuBaseline, min_seconds=5.0, max_reps=20):
        """Prompt 0 of layer 0 through the oracle's prefill, one task per query position on the
        host cores as forward.rs:927-931. Returns (baseline, the oracle's output [S][H][d])."""
        orc = cb.orc
        k, v = self.host
        st = orc.kv_cache(k[None], v[None], L=cb.L)
        q = self.q0_host[:self.S].reshape(self.S, -1)
        nt = cb.threads
        reps, t0 = 0, time.perf_counter()
        while True:
            out = orc.prefill(q, st, 0, 0, self.H, self.Hkv, self.d, self.scale, n_threads=nt)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min_seconds or reps >= max_reps:
                break
        flops = 4 * self.H * self.d * self.S * (self.S + 1) // 2 * reps
        base = dict(value=round(flops / el / 1e12, 6), unit="TFLOP/s", kind="port",
                    sample=f"{reps} x prompt 0 of layer 0 ({self.S} positions, causal), oracle prefill, one task "
                           f"per query position, {el:.1f} s")
        return cb.describe(base, nt), out.reshape(self.S, self.H, self.d)

    def gpu_sample(self):
        """Prompt 0 of layer 0 at the current precision."""
        self.step(0)
        self.be.sync()
        return self.out.download((self.B * self.S, self.H, self.d))[:self.S]

    def drop_device(self):
        self.cache.destroy()
        for buf in self.q + [self.out, self.q_start, self.pos]:
            buf.free()
        self.q = []


class ProjMatvec:
    """The Q8_0 weight matvec beside attention (gla_matvec_q8_0): Llama-3-8B's fused QKV projection
    (6144 x 4096 GGML Q8_0, 26.7 MB) for n_vec tokens, over 16 layers' weights in rotation (427 MB,
    past the 256 MB last-level cache). Synthetic GGML bytes: int8 quants uniform in [-127, 127], f16
    scales |N(0, 1)| / 127."""

    def __init__(self, be, n_vec, rows=6144, cols=4096, n_layers=16, seed=0x5151):
        self.be, self.n_vec, self.rows, self.cols = be, n_vec, rows, cols
        rng = np.random.default_rng(seed)
        nb = cols // 32
        self.w, self.raw0 = [], None
        for layer in range(n_layers):
            blk = np.empty((rows, nb, 34), np.uint8)
            blk[:, :, 2:] = rng.integers(-127, 128, (rows, nb, 32), dtype=np.int8).view(np.uint8)
            sc = (np.abs(rng.standard_normal((rows, nb))) / 127).astype(np.float16)
            blk[:, :, :2] = sc.view(np.uint8).reshape(rows, nb, 2)
            if layer == 0:
                self.raw0 = blk.reshape(-1).copy()
            self.w.append(be.create_q8_weights(blk, rows, cols))
        self.x_host = rng.standard_normal((n_vec, cols)).astype(np.float32)
        self.x = be.buffer(self.x_host)
        self.y = be.empty(n_vec * rows * 4)
        be.sync()

    def step(self, i):
        self.be.matvec_q8_0(self.w[i % len(self.w)], self.x, self.n_vec, self.y)

    def bytes_per_step(self):
        return float(self.rows * self.cols // 32 * 34 + self.n_vec * (self.cols + self.rows) * 4)

    def cpu_baseline(self, cb: CpuBaseline, min_seconds=3.0, max_reps=50):
        """One layer's QKV matvec for one token through the oracle's restatement of
        matvec_q8_0_scalar (quantized.rs:587-610), one thread. Returns (baseline, y [rows])."""
        orc = cb.orc
        reps, t0 = 0, time.perf_counter()
        while True:
            out = orc.matvec_q8_0(self.raw0, self.rows, self.cols, self.x_host[0], L=cb.L)
            reps += 1
            el = time.perf_counter() - t0
            if el >= min_seconds or reps >= max_reps:
                break
        nbytes = self.rows * self.cols // 32 * 34 * reps
        base = dict(value=round(nbytes / el / 1e9, 3), unit="GB/s", kind="port",
                    sample=f"{reps} x one token through layer 0's 6144 x 4096 weights, oracle matvec_q8_0 "
                           f"(scalar), {el:.1f} s")
        return cb.describe(base, 1), out

    def gpu_sample(self):
        """Token 0 through layer 0's weights."""
        self.step(0)
        self.be.sync()
        return self.y.download((self.n_vec, self.rows))[0]

    def drop_device(self):
        for w in self.w:
            w.destroy()
        self.w = []
        self.x.free()
        self.y.free()


def calibrate(be: GpuBackend, n_copies: int = 2048) -> dict:
    """Known-size copies for the FETCH_SIZE / WRITE_SIZE scale: gla_pool_copy_page on a
    Q8_0 pool of the cfg3 shape copies one page (34,816 bytes read and written) per dispatch."""
    pool = be.create_page_pool(2 * n_copies, 8, 128, "q8")
    for i in range(n_copies):
        pool.copy_page(i, n_copies + i)
    be.sync()
    nbytes = 8 * 34 * 128
    pool.destroy()
    return {"kernel": "copy_bytes_kernel", "dispatches": n_copies, "bytes_read_per_dispatch": nbytes,
            "bytes_written_per_dispatch": nbytes}


def traffic_from_profile() -> tuple[int | None, str | None]:
    """HBM bytes per decode call from the committed rocprofv3 counter summary, if any."""
    if not PMC_SUMMARY.exists():
        return None, None
    m = re.search(r"^traffic_bytes_per_call:\s*(\d+)", PMC_SUMMARY.read_text(), re.M)
    return (int(m.group(1)), str(PMC_SUMMARY.relative_to(ROOT))) if m else (None, None)


# --------------------------------------------------------------------------- main
def probe_lib():
    lib = C.CDLL(str(ROOT / "glint_amd" / "libglint_probe.so"))
    lib.glp_stream_read.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_double)]
    lib.glp_mfma_peak.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_double)]
    lib.glp_read_per_launch.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_int, C.c_int,
                                        C.POINTER(C.c_double)]
    lib.glp_mfma_clock.argtypes = [C.c_int, C.POINTER(C.c_double)]
    return lib


class Settle:
    """A kernel of the leg's kind right before its warmup (see the module docstring): "hbm"
    streams a 1 GiB buffer 625 times with non-temporal loads (~0.1 s at 7 TB/s); "mfma" runs
    the bf16 MFMA-only loop on random N(0,1) operands for 550,000 iterations (~0.3 s), whose
    power draw is closest to the prefill's (the near-constant-operand loop, or 0.08 s, left
    the next calls 1-3% slower)."""

    HOW = {"hbm": "625 streaming reads of a 1 GiB buffer (glp_stream_read), ~0.1 s",
           "mfma": "bf16 MFMA-only loop on random operands, 550,000 iterations (glp_mfma_peak mode 2), ~0.3 s"}

    def __init__(self, be: GpuBackend, on: bool = True):
        self.lib = probe_lib()
        self.buf = be.empty(1 << 30)
        self.on = on

    def __call__(self, kind: str) -> str:
        if not self.on:
            return "none"
        out = C.c_double()
        if kind == "hbm":
            rc = self.lib.glp_stream_read(self.buf.ptr, 1 << 30, 625, C.byref(out))
        else:
            rc = self.lib.glp_mfma_peak(2, 550000, C.byref(out))
        if rc != 0:
            raise RuntimeError(f"gla_probe settle call failed ({rc})")
        return kind

    def close(self):
        self.buf.free()


# Per-launch read ceilings: the bytes one call of a small workload must read, read by one
# launch of the streaming-read kernel (the best of these workgroup counts), launches back to
# back over a 2 GiB buffer in rotation so that each comes from HBM. "empty" is the launch floor.
PER_LAUNCH_READS = {
    "empty": (16, (1,)),
    "cfg1_call": (2 * 512 * 3 * 64 * 4, (64, 128, 256, 512)),         # K+V of one SmolLM layer, ctx 512
    "proj_qkv_weights": (6144 * 128 * 34, (256, 512, 1024, 2048)),      # Q8_0 QKV weight bytes
    "cfg2_layer": (2 * 4096 * 8 * 128 * 4, (256, 512, 1024, 2048, 4096)),  # K+V of one Llama layer, ctx 4096
}


def per_launch_reads(lib, buf, nbytes: int) -> dict:
    out = {}
    us = C.c_double()
    for name, (size, grids) in PER_LAUNCH_READS.items():
        best = None
        for wgs in grids:
            rc = lib.glp_read_per_launch(buf.ptr, nbytes, size, wgs, 200, C.byref(us))
            if rc != 0:
                raise RuntimeError(f"gla_probe glp_read_per_launch failed ({rc})")
            if best is None or us.value < best[0]:
                best = (us.value, wgs)
        out[name] = {"bytes": size, "us": round(best[0], 2), "workgroups": best[1],
                     "GB_per_s": round(size / (best[0] * 1e-6) / 1e9, 1)}
    return out


def achievable(be: GpuBackend, settle: Settle) -> dict:
    """Ceilings measured on this GPU (glint_amd/csrc/gla_probe.hip): a 2 GiB streaming read with
    non-temporal loads, one read per launch at the sizes of the small workloads
    (PER_LAUNCH_READS), and MFMA-only loops for fp32 (16x16x4) and bf16 (16x16x32), each after a
    settle of its kind."""
    lib = settle.lib
    nbytes = 2 << 30
    buf = be.empty(nbytes)
    gbs, f32, bf16, bf16r, f32r = C.c_double(), C.c_double(), C.c_double(), C.c_double(), C.c_double()
    settle("hbm")
    rc = lib.glp_stream_read(buf.ptr, nbytes, 10, C.byref(gbs))
    per_launch = per_launch_reads(lib, buf, nbytes) if rc == 0 else None
    if rc == 0:
        settle("mfma")
    mhz = C.c_double()
    for rc in (rc,
               lib.glp_mfma_peak(0, 50000, C.byref(f32)), lib.glp_mfma_peak(1, 50000, C.byref(bf16)),
               lib.glp_mfma_peak(2, 50000, C.byref(bf16r)), lib.glp_mfma_clock(50000, C.byref(mhz)),
               lib.glp_mfma_peak(3, 50000, C.byref(f32r))):
        if rc != 0:
            raise RuntimeError(f"gla_probe call failed ({rc})")
    del buf
    return {"hbm_read_gbs": round(gbs.value, 1), "fp32_mfma_tflops": round(f32.value, 1),
            "bf16_mfma_tflops": round(bf16.value, 1), "bf16_mfma_random_data_tflops": round(bf16r.value, 1),
            "fp32_mfma_random_data_tflops": round(f32r.value, 1),
            "bf16_mfma_random_data_clock_mhz": round(mhz.value), "read_per_launch": per_launch,
            "how": "2 GiB streaming read with non-temporal 16-byte loads; one read per launch of each "
                   "small workload's bytes, back to back over the 2 GiB buffer in rotation (best "
                   "workgroup count; launch gaps included); MFMA-only loops, 8 waves per CU, "
                   "8 independent accumulators per wave, on near-constant operands and on random "
                   "N(0,1) operands, and the shader clock the random-operand bf16 loop runs at "
                   "(glint_amd/csrc/gla_probe.hip); each after a settle of its kind"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "proj", "all"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs and the error figures")
    ap.add_argument("--calibrate", action="store_true", help="also run known-size page copies (for PMC runs)")
    ap.add_argument("--achievable", action="store_true",
                    help="measure the achievable ceilings also when one workload is selected")
    ap.add_argument("--no-settle", action="store_true",
                    help="no settle kernel before each leg's warmup (to measure the settle's effect)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU: the attention path has no multi-GPU leg "
                                   "(decode would shard a sequence's pages across GPUs and merge the "
                                   "log-sum-exp partials); run with --gpus 1"}))
        return 2

    be = GpuBackend(0)
    ev = HipEvents()
    cb = None if args.no_cpu else CpuBaseline()
    steps = max(20, args.steps)  # every leg: the median of at least 20 timed steps
    want = {args.workload} if args.workload != "all" else {"cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "proj"}
    result = {
        "metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (Q8_0 KV; products as exact f16 pieces on MFMA, f32 accumulate and softmax)",
        "data": "synthetic (seeded Xorshift64 + Box-Muller, N(0,1) Q/K/V; K x3 for config 5)",
    }
    secondary = {}
    ach = None
    settle = Settle(be, on=not args.no_settle)
    result["settle"] = ({"before": "each leg's warmup, after its set-up", **Settle.HOW} if settle.on
                        else {"before": "none (--no-settle)"})
    if args.workload == "all" or args.achievable:
        log("achievable ceilings (streaming read, MFMA loops)")
        ach = achievable(be, settle)
        result["achievable"] = ach

    def frac_of(value, key):
        return round(value / ach[key], 4) if ach else None

    # The CPU legs run after every GPU leg: CPU work between two GPU legs leaves the GPU idle for
    # seconds, and the next leg's timing then measured up to 7% slower (cfg4 bf16 0.182-0.186 ms
    # after the fp32 leg's CPU baseline against 0.171-0.174 ms without it, on one box). Each GPU
    # leg takes its sample's GPU output right after its timing; `place(base, ref, errors)` files
    # the CPU leg's results.
    pending = []

    def defer(wl, place, tol=(1e-4, 1e-3), **kw):
        if cb is not None:
            pending.append((wl, kw, wl.gpu_sample(), tol, place))
        wl.drop_device()  # a finished leg keeps host data only

    if "cfg3" in want:
        log("cfg3: paged Q8_0 pool, 2 layers, B=64")
        wl = PagedDecode(be, "cfg3", 32, 8, 128, 64, 128, 8192, 256, None, [None, None], 1.0, SEED + 3)
        settled = settle("hbm")
        t = time_steps(be, ev, wl.step, steps, args.warmup)
        ms = t.median_ms
        gbs = wl.bytes_per_step() / (ms * 1e-3) / 1e9
        traffic, src = traffic_from_profile()
        result.update(value=round(gbs, 2), ms_per_step=round(ms, 5))
        result["config"] = {
            "workload": "cfg3: Llama-3-8B decode attention, paged Q8_0 KV, B=64, ctx U[128,8192], 16-token pages, "
                        "256-token shared prefix; one step = one layer's gla_decode for the batch (2 layers "
                        "alternating)",
            "n_heads": 32, "n_kv_heads": 8, "head_dim": 128, "batch": 64, "kv_format": "q8_0 paged",
            "sum_ctx": int(wl.ctx.sum()), "bytes_per_step_unique": int(wl.bytes_per_step()),
            "bytes_per_step_logical": int(np.mean([L["bytes_logical"] for L in wl.layers])),
        }
        result["roofline"] = {
            "bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "achievable_peak": ach["hbm_read_gbs"] if ach else None,
            "frac_of_achievable": frac_of(gbs, "hbm_read_gbs"),
            "kernel": "decode_q8_mfma_kernel<128> + decode_q8_combine_kernel<128> (one gla_decode call)",
            "algorithmic_bytes_per_call": int(wl.bytes_per_step()),
            "us_per_call": round(ms * 1e3, 2), "timing_us": t.summary_us(), "settle": settled,
        }
        if src:
            result["roofline"]["traffic_source"] = src
        log(f"cfg3: {ms * 1e3:.1f} us/call (median; min {t.per.min() * 1e3:.1f}, max {t.per.max() * 1e3:.1f}), "
            f"{gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of peak)")
        def place_cfg3(base, ref, errors):
            result["cpu_baseline"], result["errors"] = base, errors
        defer(wl, place_cfg3)
        del wl
    if "cfg5" in want:
        log("cfg5: Gemma-2 paged Q8_0 pool (windowed + global layer)")
        wl = PagedDecode(be, "cfg5", 16, 8, 256, 32, 2048, 8192, 0, 50.0, [4096, None], 3.0, SEED + 5)
        settled = settle("hbm")
        t = time_steps(be, ev, wl.step, steps, args.warmup)
        ms = t.median_ms
        gbs = wl.bytes_per_step() / (ms * 1e-3) / 1e9
        e = secondary["cfg5"] = {
            "workload": "Gemma-2-9B decode, paged Q8_0, B=32, ctx U[2048,8192], soft-cap 50, window 4096 and "
                        "global layers alternating (one step = one layer)",
            "value": round(gbs, 2), "unit": "GB/s", "us_per_layer": round(ms * 1e3, 2), "timing_us": t.summary_us(),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "frac_of_achievable_hbm": frac_of(gbs, "hbm_read_gbs"), "settle": settled}
        defer(wl, lambda base, ref, errors, e=e: e.update(cpu_baseline=base, errors=errors),
              min_seconds=5.0, max_reps=10)
        log(f"cfg5: {ms * 1e3:.1f} us/layer, {gbs:.1f} GB/s")
        del wl
    if "cfg2" in want:
        log("cfg2: 32-layer f32 cache")
        wl = ContigDecode(be, 32, 4096, 32, 8, 128, 0x2222, "cfg2")
        settled = settle("hbm")
        t = time_steps(be, ev, wl.step, steps, args.warmup, group=wl.n_layers)
        ms = t.median_ms
        gbs = wl.bytes_per_step() / (ms * 1e-3) / 1e9
        e = secondary["cfg2"] = {
            "workload": "Llama-3-8B single-sequence decode, f32 contiguous ctx 4096, 32 layers back to back",
            "value": round(gbs, 2), "unit": "GB/s", "us_per_layer": round(ms * 1e3, 2), "timing_us": t.summary_us(),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "frac_of_achievable_hbm": frac_of(gbs, "hbm_read_gbs"), "settle": settled}
        if ach:
            e["read_per_launch_ceiling_us"] = ach["read_per_launch"]["cfg2_layer"]["us"]
        defer(wl, lambda base, ref, errors, e=e: e.update(cpu_baseline=base, errors=errors))
        log(f"cfg2: {ms * 1e3:.1f} us/layer, {gbs:.1f} GB/s")
        del wl
    if "cfg1" in want:
        log("cfg1: SmolLM-135M decode, f32 ctx 512")
        wl = ContigDecode(be, 8, 512, 9, 3, 64, 0x1111, "cfg1")
        settled = settle("hbm")
        t = time_steps(be, ev, wl.step, steps, args.warmup, group=wl.n_layers)
        ms = t.median_ms
        e = secondary["cfg1"] = {
            "workload": "SmolLM-135M decode, H9/KV3 d64, B=1, f32 contiguous ctx 512 (latency)",
            "value": round(ms * 1e3, 2), "unit": "us/call", "timing_us": t.summary_us(),
            "GB_per_s": round(wl.bytes_per_step() / (ms * 1e-3) / 1e9, 2), "settle": settled}
        if ach:
            e["read_per_launch_ceiling_us"] = ach["read_per_launch"]["cfg1_call"]["us"]
        log(f"cfg1: {ms * 1e3:.2f} us/call")
        # the same layers' calls captured as one HIP graph (a decode step's attention), replayed:
        # the launch cost of a call is then paid once per step, not once per kernel
        g = be.capture(lambda: [wl.step(i) for i in range(wl.n_layers)])
        settled = settle("hbm")
        t = time_steps(be, ev, lambda i: g.replay(), steps, args.warmup, group=4)
        ms_g = t.median_ms / wl.n_layers
        g.destroy()
        secondary["cfg1_graph"] = {
            "workload": f"cfg1, the {wl.n_layers} layers' gla_decode calls captured as one HIP graph and replayed",
            "value": round(ms_g * 1e3, 2), "unit": "us/call", "timing_us_per_replay": t.summary_us(),
            "GB_per_s": round(wl.bytes_per_step() / (ms_g * 1e-3) / 1e9, 2), "settle": settled}
        log(f"cfg1 graph: {ms_g * 1e3:.2f} us/call")
        defer(wl, lambda base, ref, errors, e=e: e.update(cpu_baseline=base, errors=errors),
              min_seconds=2.0, max_reps=20000)
        del wl
    if "cfg4" in want:
        log("cfg4: 4x2048 causal prefill, f32 KV cache")
        wl = Prefill(be)
        # bf16-input variant first: the fp32 leg's ~60 ms of full-rate MFMA work just before it
        # left its calls 2-5% slower than after its own settle alone
        wl.precision = "bf16"
        settled = settle("mfma")
        t = time_steps(be, ev, wl.step, steps, args.warmup)
        ms = t.median_ms
        tf = wl.flops_per_step() / (ms * 1e-3) / 1e12
        e_bf16 = secondary["cfg4_bf16"] = {
            "workload": "Llama-3-8B causal prefill 4x2048, f32 KV cache, bf16-input MFMA (fp32 accumulate)",
            "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "timing_us": t.summary_us(),
            "frac_of_bf16_mfma_peak": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
            "frac_of_achievable_bf16_mfma": frac_of(tf, "bf16_mfma_tflops"),
            "frac_of_achievable_bf16_mfma_random_data": frac_of(tf, "bf16_mfma_random_data_tflops"),
            "tolerance": "max abs 3e-2 / rel 3e-2 vs the fp32 oracle (tests/test_gpu_prefill.py)",
            "settle": settled}
        log(f"cfg4 bf16: {ms:.3f} ms/step, {tf:.1f} TFLOP/s")
        wl.precision = "f32"
        settled = settle("mfma")
        t = time_steps(be, ev, wl.step, steps, args.warmup)
        ms = t.median_ms
        tf = wl.flops_per_step() / (ms * 1e-3) / 1e12
        e_f32 = secondary["cfg4_f32"] = {
            "workload": "Llama-3-8B causal prefill 4x2048, f32 KV cache, fp32-input MFMA",
            "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "timing_us": t.summary_us(),
            "frac_of_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "frac_of_achievable_fp32_mfma": frac_of(tf, "fp32_mfma_tflops"),
            "frac_of_achievable_fp32_mfma_random_data": frac_of(tf, "fp32_mfma_random_data_tflops"),
            "settle": settled}
        sample_f32 = wl.gpu_sample() if cb is not None else None
        log(f"cfg4 f32: {ms:.3f} ms/step, {tf:.1f} TFLOP/s")
        # one CPU leg for both precisions (the same sample inputs): the bf16 output against the
        # fp32 oracle at the bf16 bar, the fp32 output (taken above) at the fp32 bar
        def place_cfg4(base, ref, errors, e_bf16=e_bf16, e_f32=e_f32, sample_f32=sample_f32):
            e_f32.update(cpu_baseline=base, errors=error_figures(sample_f32, ref, 1e-4, 1e-3))
            e_bf16["errors"] = errors
        wl.precision = "bf16"  # the deferred sample is the bf16 output
        defer(wl, place_cfg4, tol=(3e-2, 3e-2))
        del wl
    if "proj" in want:
        for n_vec in (1, 64):
            log(f"proj: Q8_0 QKV matvec, {n_vec} token(s)")
            wl = ProjMatvec(be, n_vec)
            settled = settle("hbm")
            t = time_steps(be, ev, wl.step, steps, args.warmup, group=len(wl.w))
            ms = t.median_ms
            gbs = wl.bytes_per_step() / (ms * 1e-3) / 1e9
            key = f"proj_qkv_b{n_vec}"
            e = secondary[key] = {
                "workload": f"Llama-3-8B fused QKV projection, 6144 x 4096 GGML Q8_0 weights (16 layers in "
                            f"rotation), {n_vec} token(s) per call (gla_matvec_q8_0)",
                "value": round(gbs, 2), "unit": "GB/s", "us_per_call": round(ms * 1e3, 2),
                "timing_us": t.summary_us(), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                "frac_of_achievable_hbm": frac_of(gbs, "hbm_read_gbs"), "settle": settled}
            if ach:  # the weights alone, read by one launch
                e["read_per_launch_ceiling_us"] = ach["read_per_launch"]["proj_qkv_weights"]["us"]
            def place_proj(base, ref, errors, e=e, n_vec=n_vec):
                e["errors"] = errors
                if n_vec == 1:
                    e["cpu_baseline"] = base
            defer(wl, place_proj)
            log(f"{key}: {ms * 1e3:.2f} us/call, {gbs:.1f} GB/s")
            del wl
    if args.calibrate:
        log("calibration copies")
        result["calibration"] = calibrate(be)
    if pending:
        log("CPU baselines and errors (oracle, same inputs as each leg's sample)")
    for wl, kw, sample, tol, place in pending:
        base, ref = wl.cpu_baseline(cb, **kw)
        place(base, ref, error_figures(sample, ref, *tol))
    pending.clear()

    if result["value"] is None:  # a single secondary workload was asked for: report it as the line
        name, s = next(iter(secondary.items()))
        result.update(value=s["value"], unit=s["unit"], ms_per_step=s.get("ms_per_step", s.get("us_per_layer", 0) / 1e3))
        result["config"] = {"workload": s["workload"]}
    if secondary:
        result["secondary"] = secondary
    print(json.dumps(result), flush=True)
    settle.close()
    be.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
