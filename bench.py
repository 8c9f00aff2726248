"""Benchmark: the non-GEMM ops of one Qwen3-4B prefill layer on one MI355X.

Workload (one step = one layer's hot path over one batch): 4 x 2048 = 8192 tokens, fp16 activations
~N(0,1): input RMSNorm [8192, 2560] -> q/k head RMSNorm + NeoX RoPE (32 q + 8 kv heads of 128,
theta 1e6, positions 0..2047 per sequence) -> post-attention RMSNorm [8192, 2560] -> SwiGLU on
gate/up [8192, 9728]. Inputs are resident in HBM before timing.

Each op is timed with HIP events (created with hipEventDisableSystemFence, so recording them does not
write back and invalidate the caches; their intervals then match rocprofv3's kernel durations) on
the stream it runs on, after a 1 GiB streaming read that
evicts L2 and the 256 MB Infinity Cache, so every op reads its operands from HBM (the flush is
outside the event pair). The sweep reads, so it leaves no dirty lines whose write-back the timed op
would pay for. The step is then timed as the layer runs it: after one flush, the four ops issued
back-to-back on the stream inside one event pair (the post-attention RMSNorm reads its own residual
buffer, so no op finds its input in a cache). value = algorithmic bytes of the four ops / the median
step time (ms_per_step, us_per_layer); us_per_layer_sum_of_ops adds the per-op medians instead (it
also counts one event pair's overhead per op, ~1.3 us). wall_ms_per_step (the barrier-to-barrier
clock of the K timed rounds, divided by K) also contains the flushes.

cpu_baseline: the reference's portable C++ ops (oracle/_ref, compiled from its sources) -- or the
oracle's C restatement where that is absent -- on f32 activations, one pinned core, over a bounded
row sample of the same workload. With --all, every op carries the same kind of figure (cpu_us).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("achieved HBM GB/s (% of 8 TB/s) per fused op; µs/layer non-GEMM ops, Qwen3-4B")
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
VALU_F32_PEAK_TFLOPS = 157.3  # MI355X fp32 vector FMA
# qwen3_4b_attention: (op, tokens, first position, first token of the CPU sample)
ATTENTION_CASES = (("decode_4k", 1, 4095, 0), ("decode_32k", 1, 32767, 0), ("prefill_2k", 2048, 0, 2032),
                   ("prefill_8k", 8192, 0, 8188))
OPS = ("rmsnorm_in", "qk_norm_rope", "rmsnorm_post", "swiglu")
DOMINANT = "swiglu"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-flush", action="store_true", help="skip the cache flush (cache-warm figures)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-floors", action="store_true", help="skip the per-op floors timed beside the ops")
    p.add_argument("--only", default=None, help="time a single op (for profiling runs)")
    p.add_argument("--all", action="store_true",
                   help="time every configured workload's ops (one JSON line with all of them) instead")
    p.add_argument("--workload", default=None,
                   help="with --all: time only this workload (gpt2_small_chain, qwen3_0.6b_decode, qwen3_4b_prefill, "
                        "qwen3_4b_prefill_f32, "
                        "quant_gather_qwen3_1.7b, qwen3_4b_fused, quantize_qwen3_1.7b_table, granite_4.0h_norms, "
                        "qwen3_4b_decode_matmul, qwen3_4b_decode4_matmul, qwen3_4b_decode16_matmul, qwen3_4b_decode24_matmul, "
                        "qwen3_4b_decode_matmul_f32, qwen3_4b_decode16_matmul_f32, "
                        "qwen3_4b_prefill_matmul, qwen3_4b_attention, stream_floor)")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="also run one plain device copy of this many MiB (calibrates rocprof byte counters)")
    return p.parse_args()


def progress(msg: str) -> None:
    """One line on stderr per finished phase, so a long run shows it is moving."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


class HipTimer:
    """Start/stop HIP event pairs on one stream, created with hipEventDisableSystemFence."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, stream: int):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.stream = ctypes.c_void_p(stream or None)
        self.events = []

    def pair(self):
        ev = []
        for _ in range(2):
            e = self.ct.c_void_p()
            if self.hip.hipEventCreateWithFlags(self.ct.byref(e), self.DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            ev.append(e)
        self.events += ev
        return ev

    def record(self, e):
        if self.hip.hipEventRecord(e, self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, s, e) -> float:
        ms = self.ct.c_float()
        if self.hip.hipEventElapsedTime(self.ct.byref(ms), s, e) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def close(self):
        for e in self.events:
            self.hip.hipEventDestroy(e)
        self.events = []


class FloorLib:
    """The streaming-floor kernels (libneko_floor.so) and the HIP runtime's own device-to-device copies
    (hipMemcpyAsync, hipMemcpy2DAsync), as zero-argument calls on one stream that raise on error."""

    H2D, D2D = 1, 3

    def __init__(self, stream: int):
        import ctypes

        c = ctypes
        self.ct = c
        self.bound = set()  # functions whose argument types are declared below
        lib = c.CDLL(os.path.join(ROOT, "nekochat_amd", "libneko_floor.so"))
        for name, args_ in (("neko_floor_empty", [c.c_int, c.c_void_p]),
                            ("neko_floor_copy", [c.c_void_p, c.c_void_p, c.c_size_t, c.c_int, c.c_int, c.c_int,
                                                 c.c_void_p]),
                            ("neko_floor_copy2", [c.c_void_p, c.c_void_p, c.c_void_p, c.c_size_t, c.c_int, c.c_int,
                                                  c.c_void_p]),
                            ("neko_floor_read", [c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p]),
                            ("neko_floor_rows2", [c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_int64, c.c_int64,
                                                  c.c_int, c.c_int, c.c_void_p]),
                            ("neko_floor_inplace", [c.c_void_p, c.c_int64, c.c_int64, c.c_int64, c.c_int, c.c_int,
                                                    c.c_void_p]),
                            ("neko_floor_inplace_rows", [c.c_void_p, c.c_int64, c.c_int64, c.c_int64, c.c_int, c.c_int,
                                                         c.c_int, c.c_void_p]),
                            ("neko_floor_rows_up", [c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_int64, c.c_int,
                                                    c.c_int, c.c_int, c.c_void_p]),
                            ("neko_floor_gather", [c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_int64, c.c_void_p,
                                                   c.c_int64, c.c_int64, c.c_int, c.c_int, c.c_void_p]),
                            ("neko_floor_add2", [c.c_void_p, c.c_void_p, c.c_void_p, c.c_size_t, c.c_int, c.c_int, c.c_int,
                                                 c.c_void_p]),
                            ("neko_floor_split2", [c.c_void_p, c.c_int64, c.c_int64, c.c_void_p, c.c_void_p, c.c_int64,
                                                   c.c_int64, c.c_void_p]),
                            ("neko_floor_inplace_kv", [c.c_void_p, c.c_int64, c.c_int64, c.c_int64, c.c_int64, c.c_void_p,
                                                       c.c_void_p, c.c_int64, c.c_void_p]),
                            ("neko_floor_gate", [c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_void_p, c.c_int64,
                                                 c.c_int64, c.c_int64, c.c_void_p]),
                            ("neko_floor_copy_x", [c.c_void_p, c.c_void_p, c.c_size_t, c.c_int, c.c_int, c.c_int, c.c_void_p]),
                            ("neko_floor_rows2_x", [c.c_void_p, c.c_int64, c.c_void_p, c.c_int64, c.c_int64, c.c_int64,
                                                    c.c_int, c.c_void_p]),
                            ("neko_floor_inplace_x", [c.c_void_p, c.c_int64, c.c_int64, c.c_int64, c.c_int, c.c_void_p])):
            getattr(lib, name).argtypes = args_
            getattr(lib, name).restype = c.c_int
            self.bound.add(name)
        self.lib = lib
        hip = c.CDLL("libamdhip64.so.7")  # the runtime torch already loaded
        hip.hipMemcpyAsync.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_int, c.c_void_p]
        hip.hipMemcpyAsync.restype = c.c_int
        hip.hipMemcpy2DAsync.argtypes = [c.c_void_p, c.c_size_t, c.c_void_p, c.c_size_t, c.c_size_t, c.c_size_t,
                                         c.c_int, c.c_void_p]
        hip.hipMemcpy2DAsync.restype = c.c_int
        self.hip = hip
        self.stream = c.c_void_p(stream or None)

    def _checked(self, fn, *a):
        stream = self.stream

        def call():
            rc = fn(*a, stream)
            if rc != 0:
                raise RuntimeError(f"{fn.__name__}: HIP error {rc}")
        return call

    def __getattr__(self, name):  # floor kernels by their exported name without the prefix
        full = "neko_floor_" + name
        if full not in self.__dict__.get("bound", ()):
            # Without declared argument types ctypes passes Python ints as 32-bit C ints: device
            # pointers would reach the kernel truncated.
            raise AttributeError(f"{full}: no argument types declared in FloorLib")
        fn = getattr(self.lib, full)
        return lambda *a: self._checked(fn, *a)

    def memcpy(self, dst, src, nbytes):
        """hipMemcpyAsync device to device."""
        return self._checked(self.hip.hipMemcpyAsync, dst, src, nbytes, self.D2D)

    def memcpy2d(self, dst, dpitch, src, spitch, width, rows):
        """hipMemcpy2DAsync device to device: `rows` rows of `width` bytes."""
        return self._checked(self.hip.hipMemcpy2DAsync, dst, dpitch, src, spitch, width, rows, self.D2D)


def headline_floors(cfg, inp, dev, fl):
    """Floor candidates for each headline op over the op's own byte pattern and data (the op's input
    tensors as the sources): the floor kernels (copies in the op's layout) and the runtime's
    device-to-device copies (hipMemcpyAsync, hipMemcpy2DAsync, torch's copy_). Returns (calls, bytes, {op: [candidate names]}, {op: {candidate: call}} for the
    layer-floor step, whose two RMSNorm floors use separate buffers so neither finds the other's bytes
    in a cache)."""
    import torch

    from nekochat_amd import workloads as wl

    calls, nbytes, groups, layer = {}, {}, {}, {}
    half = cfg.T * cfg.C * 2  # one [T, C] fp16 row set
    # the one-round row kernels' shape: every row of a wave requested before any store (at four waves
    # per SIMD: ceil(T / (16 CUs)) rows per wave), with and without a barrier between reads and writes
    r_up = -(-cfg.T // (16 * torch.cuda.get_device_properties(dev).multi_processor_count))
    row_b = cfg.C * 2
    for op in ("rmsnorm_in", "rmsnorm_post"):
        # The op's own input rows as the source, as for the other ops' floors below: uniformly random
        # bits move measurably slower than f16 activations (and constant data faster).
        src = inp["x" if op == "rmsnorm_in" else "x_post"]
        dst = torch.empty_like(src)
        cand = {
            "copy_i1_ntnt": fl.copy(src.data_ptr(), dst.data_ptr(), half, 1, 1, 1),
            "copy_i4_ntnt": fl.copy(src.data_ptr(), dst.data_ptr(), half, 4, 1, 1),
            "copy_i1_plpl": fl.copy(src.data_ptr(), dst.data_ptr(), half, 1, 0, 0),
            "copy_i4_plpl": fl.copy(src.data_ptr(), dst.data_ptr(), half, 4, 0, 0),
            "copy_i1_plpl_x128": fl.copy_x(src.data_ptr(), dst.data_ptr(), half, 0, 0, 128),
            "copy_i1_ntnt_x128": fl.copy_x(src.data_ptr(), dst.data_ptr(), half, 1, 1, 128),
            "hipMemcpyAsync": fl.memcpy(dst.data_ptr(), src.data_ptr(), half),
            "torch_copy_": (lambda d=dst, s=src: d.copy_(s)),
        }
        if r_up <= 3 and row_b % 1024 == 0 and row_b // 1024 in (5, 10):
            for sync in (0, 1):
                cand[f"rows_up_r{r_up}{'_sync' if sync else ''}"] = fl.rows_up(
                    src.data_ptr(), row_b, dst.data_ptr(), row_b, cfg.T, r_up, row_b // 1024, sync)
        layer[op] = cand
        if op == "rmsnorm_in":  # both RMSNorms move the same bytes: one set of candidates is timed
            groups["rmsnorm"] = []
            for k, v in cand.items():
                calls[f"rmsnorm:{k}"], nbytes[f"rmsnorm:{k}"] = v, 2 * half
                groups["rmsnorm"].append(f"rmsnorm:{k}")
        layer[op]["_keep"] = (src, dst)
    # q/k RoPE: 10240 of every 12288 bytes of each qkv row read and written back, in place.
    qk_w = (cfg.n_q + cfg.n_kv) * cfg.hd * 2
    rs = cfg.qkv_stride * 2
    qf = inp["qkv"].clone()
    qf2 = torch.empty_like(qf)
    waves = 16 * torch.cuda.get_device_properties(dev).multi_processor_count
    cand = {
        "inplace_rows_ntpl": fl.inplace_rows(qf.data_ptr(), rs, cfg.T, qk_w, waves, 1, 0),
        "inplace_plpl": fl.inplace(qf.data_ptr(), rs, cfg.T, qk_w, 0, 0),
        "inplace_plpl_x64": fl.inplace_x(qf.data_ptr(), rs, cfg.T, qk_w, 64),
        "inplace_plpl_x128": fl.inplace_x(qf.data_ptr(), rs, cfg.T, qk_w, 128),
        "hipMemcpy2DAsync": fl.memcpy2d(qf2.data_ptr(), rs, qf.data_ptr(), rs, qk_w, cfg.T),
    }
    layer["qk_norm_rope"] = dict(cand, _keep=(qf, qf2))
    groups["qk_norm_rope"] = []
    for k, v in cand.items():
        calls[f"qk_norm_rope:{k}"], nbytes[f"qk_norm_rope:{k}"] = v, 2 * cfg.T * qk_w
        groups["qk_norm_rope"].append(f"qk_norm_rope:{k}")
    # SwiGLU: gate and up halves of each [T, 2I] row in, [T, I] out (318 + 159 MB). The runtime's copies
    # move as many bytes in as out, so theirs is the same total (239 + 239 MB) in a 1:1 mix.
    gi = cfg.T * cfg.I * 2
    h = inp["h"]
    gout = torch.empty((cfg.T, cfg.I), dtype=torch.float16, device=dev)
    tot = 3 * gi // 2 // 16 * 16
    d1 = torch.empty(tot, dtype=torch.uint8, device=dev)
    cand = {
        "rows2_ntpl": fl.rows2(h.data_ptr(), 2 * gi // cfg.T, gout.data_ptr(), gi // cfg.T, cfg.T, gi // cfg.T, 1, 0),
        "rows2_ntpl_x128": fl.rows2_x(h.data_ptr(), 2 * gi // cfg.T, gout.data_ptr(), gi // cfg.T, cfg.T, gi // cfg.T, 128),
        "copy2_ntpl": fl.copy2(h.data_ptr(), h.data_ptr() + gi, gout.data_ptr(), gi, 1, 0),
        "hipMemcpyAsync_same_total": fl.memcpy(d1.data_ptr(), h.data_ptr(), tot),
    }
    layer["swiglu"] = dict(cand, _keep=(gout, d1))
    groups["swiglu"] = []
    for k, v in cand.items():
        calls[f"swiglu:{k}"], nbytes[f"swiglu:{k}"] = v, 3 * gi if not k.startswith("hip") else 2 * tot
        groups["swiglu"].append(f"swiglu:{k}")
    return calls, nbytes, groups, layer


def time_ops(calls, op_bytes, names, steps, warmup, flush, timer, flushes=None, tails=None):
    """Times each named op: `warmup` untimed rounds, then `steps` rounds, each op after a cache
    flush (unless flush is None) inside its own event pair. flushes: {name: buffer} replacing the flush
    buffer for those ops; tails: {name: fn} run after the op inside its event pair. Returns (per-op
    stats, wall ms/round)."""
    import torch

    flushes, tails = flushes or {}, tails or {}

    def step(record):
        for name in names:
            fl = flushes.get(name, flush)
            if fl is not None:
                fl.sum()
            if record is None:
                calls[name]()
                if name in tails:
                    tails[name]()
            else:
                s, e = record[name]
                timer.record(s)
                calls[name]()
                if name in tails:
                    tails[name]()
                timer.record(e)

    for _ in range(warmup):
        step(None)
    events = [{n: timer.pair() for n in names} for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        step(events[k])
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    per_op = {}
    for n in names:
        times_ms = [timer.elapsed_ms(*events[k][n]) for k in range(steps)]
        med = statistics.median(times_ms)
        gbs = op_bytes[n] / (med * 1e-3) / 1e9
        per_op[n] = {"us": round(med * 1e3, 3), "mean_us": round(statistics.fmean(times_ms) * 1e3, 3),
                     "bytes": op_bytes[n], "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    timer.close()
    return per_op, wall


def time_layer(calls, names, steps, warmup, flush, timer):
    """Times the layer as it runs: per step a cache flush (unless flush is None), then the named ops
    issued back-to-back inside one event pair. Returns the per-step times in ms."""
    import torch

    def step(pair):
        if flush is not None:
            flush.sum()
        if pair is not None:
            timer.record(pair[0])
        for name in names:
            calls[name]()
        if pair is not None:
            timer.record(pair[1])

    for _ in range(warmup):
        step(None)
    pairs = [timer.pair() for _ in range(steps)]
    torch.cuda.synchronize()
    for k in range(steps):
        step(pairs[k])
    torch.cuda.synchronize()
    times = [timer.elapsed_ms(*p) for p in pairs]
    timer.close()
    return times


def gpu_bench(args):
    import torch

    from nekochat_amd import ops
    from nekochat_amd import workloads as wl

    dev = torch.device("cuda:0")
    cfg = wl.QWEN3_PREFILL
    inp = wl.qwen3_prefill_inputs(cfg, dev)
    xn = torch.empty_like(inp["x"])
    xn_post = torch.empty_like(inp["x_post"])
    g = torch.empty((cfg.T, cfg.I), dtype=torch.float16, device=dev)
    # 1 GiB swept by a sum: longer than the host needs to queue the next op, so the GPU never waits
    # for Python between the start event and the kernel.
    flush = torch.ones(256 << 20, dtype=torch.float32, device=dev)

    # Each op validated once; the timed window holds one direct C-ABI call.
    calls = {
        "rmsnorm_in": ops.prepare(ops.rms_norm, inp["x"], inp["w_in"], cfg.eps, out=xn)[0],
        "qk_norm_rope": ops.prepare(ops.qk_norm_rope, inp["qkv"], cfg.n_q, cfg.n_kv, cfg.hd, inp["cs"], cfg.eps,
                                    wqk=inp["wqk"], positions=inp["positions"])[0],
        "rmsnorm_post": ops.prepare(ops.rms_norm, inp["x_post"], inp["w_post"], cfg.eps, out=xn_post)[0],
        "swiglu": ops.prepare(ops.silu_mul, inp["h"], out=g)[0],
    }
    names = [args.only] if args.only else list(OPS)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        flush.sum()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    timer = HipTimer(torch.cuda.current_stream().cuda_stream)
    per_op, wall = time_ops(calls, cfg.op_bytes(), names, args.steps, args.warmup,
                            None if args.no_flush else flush, timer)
    progress("ops timed")
    layer = None
    floors = None
    if not args.only:
        layer = time_layer(calls, names, args.steps, args.warmup, None if args.no_flush else flush,
                           HipTimer(torch.cuda.current_stream().cuda_stream))
        progress("layer step timed")
        if not args.no_floors:
            floors = time_floors(cfg, inp, dev, args, None if args.no_flush else flush)
            progress("floors timed")
    return cfg, per_op, wall, layer, floors


def time_floors(cfg, inp, dev, args, flush):
    """Per-op floors measured in the same run as the ops, under the same events and flush: every
    candidate of headline_floors timed in its own rounds, the fastest per op taken as that op's floor,
    and the layer-floor step (the four ops' fastest floors back-to-back after one flush, one event
    pair, as the layer step is timed)."""
    import torch

    stream = torch.cuda.current_stream().cuda_stream
    fl = FloorLib(stream)
    calls, nbytes, groups, layer_cands = headline_floors(cfg, inp, dev, fl)
    per, _ = time_ops(calls, nbytes, list(calls), args.steps, args.warmup, flush, HipTimer(stream))
    best = {op: min(names, key=lambda n: per[n]["us"]) for op, names in groups.items()}
    op_group = {"rmsnorm_in": "rmsnorm", "rmsnorm_post": "rmsnorm", "qk_norm_rope": "qk_norm_rope", "swiglu": "swiglu"}
    step_calls = {op: layer_cands[op][best[op_group[op]].split(":", 1)[1]] for op in OPS}
    step = time_layer(step_calls, list(OPS), args.steps, args.warmup, flush, HipTimer(stream))
    torch.cuda.synchronize()
    return {"candidates_us": {n: per[n]["us"] for n in calls},
            "best": {op: {"kind": best[g].split(":", 1)[1], "us": per[best[g]]["us"]} for op, g in op_group.items()},
            "layer_step_us": round(statistics.median(step) * 1e3, 3)}


def _pin_one_core():
    """Pins the calling thread to its first allowed core; returns the previous mask."""
    try:
        mask = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {sorted(mask)[0]})
        return mask
    except (AttributeError, OSError):
        return None


def _unpin(mask):
    if mask is not None:
        os.sched_setaffinity(0, mask)


def _f32(shape, mean, std, stream):
    """Host f32 activations with the same generator as the device inputs (fp16-rounded values)."""
    from nekochat_amd import workloads as wl

    return wl.normal_f16(shape, mean, std, stream, "cpu").float().numpy()


class CpuLeg:
    """The reference's CPU path beside each device op of --all: its compiled ops (oracle/_ref, built
    from its sources) on f32 activations as its CPU forward passes hold them, one pinned core, a
    bounded sample of the workload's rows, median of `reps`, scaled to the full workload. An op whose
    reference form exists only inside a GEMM epilogue is timed as the oracle's restatement ("port")."""

    def __init__(self, reps: int = 3):
        from oracle import oracle as O

        self.O = O
        self.R = O.ref() if O.ref_available() else None
        self.reps = reps
        self.jobs = []

    def add(self, label, op, make, scale, sample, port=False):
        """make() builds the sample's inputs and returns (run_once, release or None)."""
        self.jobs.append((label, op, make, scale, sample, port))

    def run(self, out):
        if self.R is None:
            for label, op, *_ in self.jobs:
                out[label]["ops"][op]["cpu_kind"] = "not run: oracle/_ref (the compiled reference ops) is not built"
            return
        for label, op, make, scale, sample, port in self.jobs:
            fn, release = make()
            mask = _pin_one_core()
            fn()
            samples = []
            for _ in range(self.reps):
                t0 = time.perf_counter()
                fn()
                samples.append(time.perf_counter() - t0)
            _unpin(mask)
            if release is not None:
                release()
            us = statistics.median(samples) * scale * 1e6
            d = out[label]["ops"][op]
            d["cpu_us"] = round(us, 1)
            d["cpu_kind"] = "port" if port else "reference"
            d["cpu_sample"] = sample
            d["speedup_vs_cpu"] = round(us / d["us"], 1)


def add_cpu_jobs(leg, want):
    """Registers the CPU counterpart of every device op that all_configs times."""
    import numpy as np

    from nekochat_amd import ops
    from nekochat_amd import workloads as wl

    O, R, P = leg.O, leg.R, leg.O._ptr
    core = f"1 pinned core of {os.cpu_count()}, g++ -O3 portable x86-64 build, f32 activations"

    def every(what):
        return f"{what}; {core}"

    def rows_of(n, total):
        return f"{n} of {total} rows (median of {leg.reps}), scaled to all {total}; {core}"

    def gpt2_jobs():  # gpt2_small_chain
        c = wl.GPT2_CHAIN

        def gather():
            table = wl.normal_f16((c.vocab, c.C), 0.0, 0.02, 41, "cpu").numpy().view(np.uint8).copy()
            h = R.ref_qmatrix_new(ops.FMT_F16, c.vocab, c.C, P(table))
            del table
            ids = wl.uniform_ids(c.T, c.vocab, 43)
            wpe = _f32((c.n_ctx, c.C), 0.0, 0.02, 42)[:c.T].copy()
            x = np.empty((c.T, c.C), np.float32)
            return (lambda: R.ref_qmatrix_gather(h, P(ids), c.T, P(wpe), P(x))), (lambda: R.ref_qmatrix_free(h))

        def layernorm():
            x = _f32((c.T, c.C), 0.0, 1.0, 46)
            g, b = wl.weight_f32(c.C, 1.0, 0.02, 44, "cpu").numpy(), wl.weight_f32(c.C, 0.0, 0.02, 45, "cpu").numpy()
            y = np.empty_like(x)
            return (lambda: R.ref_layernorm(P(x), P(y), P(g), P(b), c.T, c.C, c.eps)), None

        def gelu():
            x = _f32((c.T, c.F), 0.0, 1.0, 46)
            y = np.empty_like(x)
            return (lambda: R.ref_gelu_n(P(x), P(y), x.size)), None

        leg.add("gpt2_small_chain", "gather_wte_wpe", gather, 1, every("all 128 tokens: dequantizeRow + wpe add"))
        leg.add("gpt2_small_chain", "layernorm", layernorm, 1, every("all 128 rows"))
        leg.add("gpt2_small_chain", "gelu", gelu, 1, every("all 128 x 3072 values"))

    def rms_job(T, C, eps, stream):
        def make():
            x = _f32((T, C), 0.0, 1.0, stream)
            w = wl.weight_f32(C, 1.0, 0.05, stream + 1, "cpu").numpy()
            y = np.empty_like(x)
            return (lambda: R.ref_rmsnorm(P(x), P(y), P(w), T, C, eps)), None
        return make

    def swiglu_job(T, I, stream):
        def make():
            h = _f32((T, 2 * I), 0.0, 1.0, stream)
            o = np.empty((T, I), np.float32)
            return (lambda: R.ref_silu_mul(P(h), P(o), T, I)), None
        return make

    def qk_state(T, n_q, n_kv, hd, theta, n_pos, pos, stream):
        stride = (n_q + 2 * n_kv) * hd
        qkv = _f32((T, stride), 0.0, 1.0, stream)
        wqk = wl.weight_f32(2 * hd, 1.0, 0.05, stream + 1, "cpu").numpy()
        wq, wk = wqk[:hd].copy(), wqk[hd:].copy()
        cs = O.rope_table(theta, hd, n_pos)
        return stride, qkv, wq, wk, cs, np.ascontiguousarray(pos, dtype=np.int32)

    def qk_job(T, n_q, n_kv, hd, theta, n_pos, pos, eps, stream):
        def make():
            stride, qkv, wq, wk, cs, p = qk_state(T, n_q, n_kv, hd, theta, n_pos, pos, stream)
            return (lambda: R.ref_qk_norm_rope(P(qkv), stride, T, n_q, n_kv, hd, P(p), P(wq), P(wk), P(cs), eps)), None
        return make

    def decode_jobs():  # qwen3_0.6b_decode
        c = wl.QWEN3_DECODE
        pos = wl.uniform_ids(c.T, c.n_pos, 7)
        full = every("all 64 rows")
        leg.add("qwen3_0.6b_decode", "rmsnorm", rms_job(c.T, c.C, c.eps, 1), 1, full)
        leg.add("qwen3_0.6b_decode", "qk_norm_rope", qk_job(c.T, c.n_q, c.n_kv, c.hd, c.theta, c.n_pos, pos, c.eps, 4),
                1, every("all 64 rows: per-token q/k rmsNorm + rope"))
        leg.add("qwen3_0.6b_decode", "swiglu", swiglu_job(c.T, c.I, 6), 1, full)

    def prefill_jobs(label="qwen3_4b_prefill"):  # qwen3_4b_prefill, qwen3_4b_prefill_f32 (the same f32 CPU ops)
        c, n = wl.QWEN3_PREFILL, 256
        s = rows_of(n, c.T)
        pos = np.arange(n) % c.seq
        leg.add(label, "rmsnorm_in", rms_job(n, c.C, c.eps, 1), c.T / n, s)
        leg.add(label, "qk_norm_rope", qk_job(n, c.n_q, c.n_kv, c.hd, c.theta, c.seq, pos, c.eps, 4), c.T / n, s)
        leg.add(label, "rmsnorm_post", rms_job(n, c.C, c.eps, 1), c.T / n, s)
        leg.add(label, "swiglu", swiglu_job(n, c.I, 6), c.T / n, s)

    def gather_jobs():  # quant_gather_qwen3_1.7b
        c, n = wl.QUANT_GATHER, 2048
        ids = wl.zipf_ids(c.T, c.vocab, c.s, 32)[:n].copy()
        held = {}

        def gather(fmt):
            def make():
                if "src" not in held:
                    held["src"] = _f32((c.vocab, c.C), 0.0, 0.02, 31)
                tab, used = ops.quantize_rows(fmt, held["src"])
                h = R.ref_qmatrix_new(used, c.vocab, c.C, P(tab))
                del tab
                x = np.empty((n, c.C), np.float32)
                if fmt == ops.FMT_FP4:
                    held.clear()
                return (lambda: R.ref_qmatrix_gather(h, P(ids), n, None, P(x))), (lambda: R.ref_qmatrix_free(h))
            return make

        s = f"first {n} of the {c.T} Zipf ids (median of {leg.reps}), scaled to all {c.T}; {core}"
        for fmt, name in ((ops.FMT_F16, "gather_fp16"), (ops.FMT_FP8, "gather_fp8"), (ops.FMT_FP4, "gather_fp4")):
            leg.add("quant_gather_qwen3_1.7b", name, gather(fmt), c.T / n, s)

    def fused_jobs():  # qwen3_4b_fused
        c, n = wl.QWEN3_PREFILL, 256
        s = rows_of(n, c.T)
        pos = np.arange(n)
        kw = c.n_kv * c.hd
        koff, voff = c.n_q * c.hd, (c.n_q + c.n_kv) * c.hd

        def add_rms():
            x = _f32((n, c.C), 0.0, 1.0, 71)
            d = _f32((n, c.C), 0.0, 0.5, 72)
            w = wl.weight_f32(c.C, 1.0, 0.05, 73, "cpu").numpy()
            xn = np.empty_like(x)
            return (lambda: O.lib().oracle_add_rmsnorm(P(x), P(d), P(xn), P(w), n, c.C, c.eps)), None

        def qk_kv(with_rope, with_store):
            def make():
                stride, qkv, wq, wk, cs, p = qk_state(n, c.n_q, c.n_kv, c.hd, 1e6, n, pos, 74)
                kc = np.empty((n, kw), np.uint16)
                vc = np.empty_like(kc)

                def once():
                    if with_rope:
                        R.ref_qk_norm_rope(P(qkv), stride, n, c.n_q, c.n_kv, c.hd, P(p), P(wq), P(wk), P(cs), c.eps)
                    if with_store:
                        R.ref_store_kv(P(qkv[:, koff:]), P(qkv[:, voff:]), stride, P(kc), P(vc), kw, n, 0)
                return once, None
            return make

        leg.add("qwen3_4b_fused", "add_rmsnorm", add_rms, c.T / n,
                rows_of(n, c.T) + "; the reference adds the residual in its output GEMM's epilogue, so the "
                "oracle's restatement of add + rmsNorm is timed", port=True)
        leg.add("qwen3_4b_fused", "qk_norm_rope_kv", qk_kv(True, True), c.T / n, s + ": q/k loop, then storeKv")
        leg.add("qwen3_4b_fused", "qk_norm_rope", qk_kv(True, False), c.T / n, s)
        leg.add("qwen3_4b_fused", "store_kv", qk_kv(False, True), c.T / n, s + ": storeKv")

    def attention_jobs():  # qwen3_4b_attention
        c = wl.QWEN3_PREFILL
        H, KV, hd = c.n_q, c.n_kv, c.hd

        def make(T, pos0, t0):  # the workload's tokens t0 .. T-1 (positions pos0 + t0 ..) through cpu::attention
            def mk():
                n = T - t0
                q = _f32((n, H * hd), 0.0, 1.0, 101)
                kc = _f32((pos0 + T, KV * hd), 0.0, 1.0, 102).astype(np.float16).view(np.uint16)
                vc = _f32((pos0 + T, KV * hd), 0.0, 1.0, 103).astype(np.float16).view(np.uint16)
                o = np.empty((n, H * hd), np.float32)
                return (lambda: R.ref_attention(P(q), H * hd, P(kc), P(vc), P(o), n, H, KV, hd, pos0 + t0)), None
            return mk

        for name, T, pos0, t0 in ATTENTION_CASES:
            pairs = T * pos0 + T * (T + 1) // 2  # (token, key) pairs of the whole call
            sample = sum(pos0 + t + 1 for t in range(t0, T))
            what = (f"the last {T - t0} of {T} tokens (median of {leg.reps}), scaled by (token, key) pairs to all {T}"
                    if t0 else f"all {T} token(s) (median of {leg.reps})")
            leg.add("qwen3_4b_attention", name, make(T, pos0, t0), pairs / sample,
                    f"{what} through cpu::attention on a one-thread pool; {core}")

    def quantize_jobs():  # quantize_qwen3_1.7b_table
        c, n = wl.QUANT_GATHER, 512

        def quant(fmt):
            def make():
                src = _f32((n, c.C), 0.0, 0.02, 31)
                dst = np.empty((n, O.quant_row_bytes(fmt, c.C)), np.uint8)
                return (lambda: R.ref_quantize_rows(fmt, n, c.C, P(src), P(dst))), None
            return make

        s = (f"{n} of {c.vocab} rows (median of {leg.reps}), scaled to all {c.vocab}; quantizeMatrix with no "
             f"thread pool; {core}")
        for fmt, name in ((ops.FMT_F16, "quantize_fp16"), (ops.FMT_FP8, "quantize_fp8"), (ops.FMT_FP4, "quantize_fp4")):
            leg.add("quantize_qwen3_1.7b_table", name, quant(fmt), c.vocab / n, s)

    def granite_jobs():  # granite_4.0h_norms
        c, n = wl.GRANITE_NORMS, 512
        s = rows_of(n, c.T)

        def gated():
            y = _f32((n, c.D), 0.0, 1.0, 53)
            z = _f32((n, c.D), 0.0, 1.0, 54)
            w = wl.weight_f32(c.D, 1.0, 0.05, 55, "cpu").numpy()
            return (lambda: R.ref_gated_rmsnorm(P(y), P(z), P(w), n, c.D, c.groups, c.eps)), None

        leg.add("granite_4.0h_norms", "rmsnorm", rms_job(n, c.C, c.eps, 51), c.T / n, s)
        leg.add("granite_4.0h_norms", "gated_rmsnorm", gated, c.T / n, s + ": y *= silu(z), then rmsNorm per group")
        leg.add("granite_4.0h_norms", "swiglu", swiglu_job(n, c.I, 56), c.T / n, s)

    def matmul_jobs(label, c):  # qwen3_4b_decode_matmul and its 4-, 16- and 24-sequence forms
        n = 256

        def mm(fmt, N, K):
            def make():
                src = _f32((n, K), 0.0, 0.02, 81)
                tab, used = ops.quantize_rows(fmt, src)
                h = R.ref_qmatrix_new(used, n, K, P(tab))
                x = _f32((c.T, K), 0.0, 1.0, 82)
                y = np.zeros((c.T, n), np.float32)
                return (lambda: R.ref_qmatrix_matmul(h, P(x), c.T, None, P(y), 0)), (lambda: R.ref_qmatrix_free(h))
            return make

        for pname, N, K in c.projections:
            for fmt, fname in ((ops.FMT_F16, "f16"), (ops.FMT_FP8, "fp8"), (ops.FMT_FP4, "fp4")):
                leg.add(label, f"{pname}_{fname}", mm(fmt, N, K), N / n,
                        f"{n} of {N} weight rows through cpu::matmul on a one-thread pool (median of {leg.reps}), "
                        f"scaled to all {N}; {core}")

    def prefill_matmul_jobs():  # qwen3_4b_prefill_matmul
        c, n = wl.QWEN3_PREFILL_MATMUL, 4

        def mm(fmt, N, K):
            def make():
                src = _f32((N, K), 0.0, 0.02, 91)
                tab, used = ops.quantize_rows(fmt, src)
                h = R.ref_qmatrix_new(used, N, K, P(tab))
                del tab, src
                x = _f32((n, K), 0.0, 1.0, 92)
                y = np.zeros((n, N), np.float32)
                return (lambda: R.ref_qmatrix_matmul(h, P(x), n, None, P(y), 0)), (lambda: R.ref_qmatrix_free(h))
            return make

        for pname, N, K in c.projections:
            for fmt, fname in ((ops.FMT_F16, "f16"), (ops.FMT_FP8, "fp8"), (ops.FMT_FP4, "fp4")):
                leg.add("qwen3_4b_prefill_matmul", f"{pname}_{fname}", mm(fmt, N, K), c.T / n,
                        f"{n} of {c.T} tokens through cpu::matmul on a one-thread pool (median of {leg.reps}), "
                        f"scaled to all {c.T}; {core}")

    # Each workload in its own scope: the closures above read their configuration when they run.
    for label, jobs in (
            ("gpt2_small_chain", gpt2_jobs),
            ("qwen3_0.6b_decode", decode_jobs),
            ("qwen3_4b_prefill", prefill_jobs),
            ("qwen3_4b_prefill_f32", lambda: prefill_jobs("qwen3_4b_prefill_f32")),
            ("quant_gather_qwen3_1.7b", gather_jobs),
            ("qwen3_4b_fused", fused_jobs),
            ("quantize_qwen3_1.7b_table", quantize_jobs),
            ("granite_4.0h_norms", granite_jobs),
            ("qwen3_4b_decode_matmul", lambda: matmul_jobs("qwen3_4b_decode_matmul", wl.QWEN3_DECODE_MATMUL)),
            ("qwen3_4b_decode4_matmul", lambda: matmul_jobs("qwen3_4b_decode4_matmul", wl.QWEN3_DECODE4_MATMUL)),
            ("qwen3_4b_decode16_matmul", lambda: matmul_jobs("qwen3_4b_decode16_matmul", wl.QWEN3_DECODE16_MATMUL)),
            ("qwen3_4b_decode24_matmul", lambda: matmul_jobs("qwen3_4b_decode24_matmul", wl.QWEN3_DECODE24_MATMUL)),
            ("qwen3_4b_decode_matmul_f32", lambda: matmul_jobs("qwen3_4b_decode_matmul_f32", wl.QWEN3_DECODE_MATMUL)),
            ("qwen3_4b_decode16_matmul_f32",
             lambda: matmul_jobs("qwen3_4b_decode16_matmul_f32", wl.QWEN3_DECODE16_MATMUL)),
            ("qwen3_4b_prefill_matmul", prefill_matmul_jobs),
            ("qwen3_4b_attention", attention_jobs),
    ):
        if want(label):
            jobs()


def all_configs(args):
    """Every configured workload's ops, timed the same way (reported beside the headline line)."""
    import numpy as np
    import torch

    from nekochat_amd import ops
    from nekochat_amd import workloads as wl

    dev = torch.device("cuda:0")
    flush = torch.ones(256 << 20, dtype=torch.float32, device=dev)
    out = {}
    if args.copy_mib:  # one plain device copy of known size: calibrates rocprof byte counters
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        flush.sum()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    labels = ("gpt2_small_chain", "qwen3_0.6b_decode", "qwen3_4b_prefill", "qwen3_4b_prefill_f32", "quant_gather_qwen3_1.7b",
              "qwen3_4b_fused",
              "quantize_qwen3_1.7b_table", "granite_4.0h_norms", "qwen3_4b_decode_matmul", "qwen3_4b_decode4_matmul",
              "qwen3_4b_decode16_matmul", "qwen3_4b_decode24_matmul", "qwen3_4b_decode_matmul_f32",
              "qwen3_4b_decode16_matmul_f32", "qwen3_4b_prefill_matmul", "qwen3_4b_attention", "stream_floor")
    if args.workload is not None and args.workload not in labels:
        raise SystemExit(f"bench.py: unknown workload {args.workload!r}; one of {', '.join(labels)}")

    def want(label):
        return args.workload is None or args.workload == label

    def run(label, calls, op_bytes, workload, op_flops=None, floors=None):
        """Times `calls` round-robin; floors: {op: [names of floor candidates among calls]} -- each op
        then carries the fastest as floor_us / floor_kind / over_floor."""
        progress(f"timing {label}")
        timer = HipTimer(torch.cuda.current_stream().cuda_stream)
        per_op, _ = time_ops(calls, op_bytes, list(calls), args.steps, args.warmup, flush, timer)
        for n, f in (op_flops or {}).items():  # MFMA-bound ops: their roofline is the dense f16 peak
            tf = f / (per_op[n]["us"] * 1e-6) / 1e12
            per_op[n].update({"flops": f, "TFLOPs": round(tf, 1), "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)})
        for n, cands in (floors or {}).items():
            best = min(cands, key=lambda f: per_op[f]["us"])
            per_op[n].update({"floor_us": per_op[best]["us"], "floor_kind": best,
                              "over_floor": round(per_op[n]["us"] / per_op[best]["us"] - 1, 4)})
        out[label] = {"workload": workload, "ops": per_op}
        torch.cuda.synchronize()

    # GPT-2 small chain: wte+wpe gather [128, 768] -> LayerNorm -> GELU [128, 3072]
    if want("gpt2_small_chain"):
        c1 = wl.GPT2_CHAIN
        wte = wl.normal_f16((c1.vocab, c1.C), 0.0, 0.02, 41, dev)
        wpe = wl.normal_f16((c1.n_ctx, c1.C), 0.0, 0.02, 42, dev)
        ids = torch.from_numpy(wl.uniform_ids(c1.T, c1.vocab, 43)).to(dev)
        table = wte.view(torch.uint8).reshape(c1.vocab, 2 * c1.C)
        x1 = torch.empty((c1.T, c1.C), dtype=torch.float16, device=dev)
        g1, b1 = wl.weight_f32(c1.C, 1.0, 0.02, 44, dev), wl.weight_f32(c1.C, 0.0, 0.02, 45, dev)
        y1 = torch.empty_like(x1)
        h1 = wl.normal_f16((c1.T, c1.F), 0.0, 1.0, 46, dev)
        o1 = torch.empty_like(h1)
        run("gpt2_small_chain", {
            "gather_wte_wpe": ops.prepare(ops.embed, ids, table, ops.FMT_F16, c1.C, wpe=wpe, out=x1)[0],
            "layernorm": ops.prepare(ops.layer_norm, x1, g1, b1, c1.eps, out=y1)[0],
            "gelu": ops.prepare(ops.gelu, h1, out=o1)[0],
        }, {"gather_wte_wpe": wl.bytes_gather(c1.T, 2 * c1.C, c1.C, wpe=True),
            "layernorm": wl.bytes_layernorm(c1.T, c1.C), "gelu": wl.bytes_gelu(c1.T * c1.F)},
            "GPT-2 small: gather wte+wpe [128,768], LayerNorm [128,768], GELU-tanh [128,3072]")

    # Qwen3-0.6B decode batch
    if want("qwen3_0.6b_decode"):
        c2 = wl.QWEN3_DECODE
        stride2 = (c2.n_q + 2 * c2.n_kv) * c2.hd
        x2 = wl.normal_f16((c2.T, c2.C), 0.0, 1.0, 1, dev)
        w2 = wl.weight_f32(c2.C, 1.0, 0.05, 2, dev)
        y2 = torch.empty_like(x2)
        qkv2 = wl.normal_f16((c2.T, stride2), 0.0, 1.0, 4, dev)
        wqk2 = wl.weight_f32(2 * c2.hd, 1.0, 0.05, 5, dev)
        pos2 = torch.from_numpy(wl.uniform_ids(c2.T, c2.n_pos, 7)).to(dev)
        cs2 = torch.from_numpy(ops.rope_table(c2.theta, c2.hd, c2.n_pos)).to(dev)
        h2 = wl.normal_f16((c2.T, 2 * c2.I), 0.0, 1.0, 6, dev)
        o2 = torch.empty((c2.T, c2.I), dtype=torch.float16, device=dev)
        run("qwen3_0.6b_decode", {
            "rmsnorm": ops.prepare(ops.rms_norm, x2, w2, c2.eps, out=y2)[0],
            "qk_norm_rope": ops.prepare(ops.qk_norm_rope, qkv2, c2.n_q, c2.n_kv, c2.hd, cs2, c2.eps, wqk=wqk2,
                                        positions=pos2)[0],
            "swiglu": ops.prepare(ops.silu_mul, h2, out=o2)[0],
        }, {"rmsnorm": wl.bytes_rmsnorm(c2.T, c2.C), "qk_norm_rope": wl.bytes_qk_rope(c2.T, c2.n_q, c2.n_kv, c2.hd),
            "swiglu": wl.bytes_swiglu(c2.T, c2.I)},
            "Qwen3-0.6B decode: 64 rows, RMSNorm 1024, q/k RoPE 16q+8kv x 128 at random positions, SwiGLU I=3072")

    # The streaming floor: kernels that only move bytes, timed exactly as the ops are.
    if want("stream_floor"):
        progress("timing stream_floor")
        out["stream_floor"] = stream_floor(args, flush, time_ops)

    # Qwen3-4B prefill (the headline layer)
    if want("qwen3_4b_prefill"):
        cfg, per_op, _, layer, floors = gpu_bench(argparse.Namespace(only=None, copy_mib=0, steps=args.steps,
                                                                     warmup=args.warmup, no_flush=False, no_floors=False))
        for op, d in per_op.items():
            b = floors["best"][op]
            d.update({"floor_us": b["us"], "floor_kind": b["kind"], "over_floor": round(d["us"] / b["us"] - 1, 4)})
        out["qwen3_4b_prefill"] = {"workload": "Qwen3-4B prefill layer (headline)", "ops": per_op,
                                   "layer_step_us": round(statistics.median(layer) * 1e3, 3),
                                   "layer_floor_us": floors["layer_step_us"]}

    # The headline layer's four ops on f32 activations, the type the reference's ComputeBackend (and so
    # the C++ adapter) passes: twice the activation bytes, the same kernels instantiated for f32.
    if want("qwen3_4b_prefill_f32"):
        c6 = wl.QWEN3_PREFILL
        inp = wl.qwen3_prefill_inputs(c6, dev)
        x6, xp6, qkv6, h6 = (inp[k].float() for k in ("x", "x_post", "qkv", "h"))
        y6, yp6 = torch.empty_like(x6), torch.empty_like(xp6)
        o6 = torch.empty((c6.T, c6.I), dtype=torch.float32, device=dev)
        run("qwen3_4b_prefill_f32", {
            "rmsnorm_in": ops.prepare(ops.rms_norm, x6, inp["w_in"], c6.eps, out=y6)[0],
            "qk_norm_rope": ops.prepare(ops.qk_norm_rope, qkv6, c6.n_q, c6.n_kv, c6.hd, inp["cs"], c6.eps,
                                        wqk=inp["wqk"], positions=inp["positions"])[0],
            "rmsnorm_post": ops.prepare(ops.rms_norm, xp6, inp["w_post"], c6.eps, out=yp6)[0],
            "swiglu": ops.prepare(ops.silu_mul, h6, out=o6)[0],
        }, {"rmsnorm_in": wl.bytes_rmsnorm(c6.T, c6.C, 4), "rmsnorm_post": wl.bytes_rmsnorm(c6.T, c6.C, 4),
            "qk_norm_rope": wl.bytes_qk_rope(c6.T, c6.n_q, c6.n_kv, c6.hd, e=4),
            "swiglu": wl.bytes_swiglu(c6.T, c6.I, 4)},
            "Qwen3-4B prefill layer's non-GEMM ops on f32 activations (the ComputeBackend's type): 2x RMSNorm "
            "[8192,2560], q/k RMSNorm+NeoX RoPE (32q+8kv x 128), SwiGLU [8192,9728]")
        del inp, x6, xp6, qkv6, h6, y6, yp6, o6

    # Quantised gather: 151936 x 2048 tied table, 16384 Zipf(1.1) ids, FP16 / FP8 / FP4 rows
    if want("quant_gather_qwen3_1.7b"):
        c4 = wl.QUANT_GATHER
        src = wl.normal_f16((c4.vocab, c4.C), 0.0, 0.02, 31, dev).float().cpu().numpy()
        ids4 = wl.zipf_ids(c4.T, c4.vocab, c4.s, 32)
        ids4_t = torch.from_numpy(ids4).to(dev)
        o4 = torch.empty((c4.T, c4.C), dtype=torch.float16, device=dev)
        calls4, bytes4 = {}, {}
        unique = int(np.unique(ids4).size)
        # The floor of each gather's byte pattern: the same table rows read through the same ids, the
        # same 4 KB output rows written, nothing decoded (1, 2 or 4 tokens per wave, non-temporal or plain
        # row loads -- plain ones let repeated ids hit in L2, as the op's do; the fastest counts).
        fl4 = FloorLib(torch.cuda.current_stream().cuda_stream)
        fo4 = torch.empty_like(o4)
        floor_names = {}
        for fmt, name in ((ops.FMT_F16, "gather_fp16"), (ops.FMT_FP8, "gather_fp8"), (ops.FMT_FP4, "gather_fp4")):
            tab, _ = ops.quantize_rows(fmt, src)
            tab_t = torch.from_numpy(tab).to(dev)
            calls4[name] = ops.prepare(ops.embed, ids4_t, tab_t, fmt, c4.C, out=o4)[0]
            bytes4[name] = wl.bytes_gather(c4.T, tab.shape[1], c4.C)
            calls4[name].table = tab_t  # keep the table alive with its call
            rb = tab.shape[1]
            floor_names[name] = []
            for tpw in (1, 2, 4):
                for ntl in (1, 0):
                    fname = f"floor_{name}_tpw{tpw}_{'nt' if ntl else 'pl'}"
                    calls4[fname] = fl4.gather(ids4_t.data_ptr(), c4.T, tab_t.data_ptr(), rb, rb, fo4.data_ptr(),
                                               c4.C * 2, c4.C * 2, tpw, ntl)
                    bytes4[fname] = bytes4[name]
                    floor_names[name].append(fname)
        del src
        run("quant_gather_qwen3_1.7b", calls4, bytes4,
            f"Qwen3-1.7B tied table 151936x2048, 16384 Zipf(1.1) ids ({unique} unique rows): mostly cache-served")
        ops4 = out["quant_gather_qwen3_1.7b"]["ops"]
        for name, fnames in floor_names.items():
            best = min(fnames, key=lambda f: ops4[f]["us"])
            ops4[name].update({"floor_us": ops4[best]["us"], "floor_kind": best,
                               "over_floor": round(ops4[name]["us"] / ops4[best]["us"] - 1, 4)})

    # The Qwen3-4B layer's fused neighbours: residual add + RMSNorm [8192, 2560], and q/k RoPE fused
    # with the KV-cache store for one 8192-token sequence (positions 0..8191), beside the unfused
    # q/k RoPE and KV store they replace.
    if want("qwen3_4b_fused"):
        c6 = wl.QWEN3_PREFILL
        x6 = wl.normal_f16((c6.T, c6.C), 0.0, 1.0, 71, dev)
        d6 = wl.normal_f16((c6.T, c6.C), 0.0, 0.5, 72, dev)
        w6 = wl.weight_f32(c6.C, 1.0, 0.05, 73, dev)
        xn6 = torch.empty_like(x6)
        qkv6 = wl.normal_f16((c6.T, c6.qkv_stride), 0.0, 1.0, 74, dev)
        wqk6 = wl.weight_f32(2 * c6.hd, 1.0, 0.05, 75, dev)
        cs6 = torch.from_numpy(ops.rope_table(1e6, c6.hd, c6.T)).to(dev)
        pos6 = torch.arange(c6.T, dtype=torch.int32, device=dev)
        kw6 = c6.n_kv * c6.hd
        kc6 = torch.empty((c6.T, kw6), dtype=torch.float16, device=dev)
        vc6 = torch.empty_like(kc6)
        qoff = c6.n_q * c6.hd
        calls6 = {
            "add_rmsnorm": ops.prepare(ops.add_rms_norm, x6, d6, w6, c6.eps, out=xn6)[0],
            "qk_norm_rope_kv": ops.prepare(ops.qk_norm_rope_kv, qkv6, c6.n_q, c6.n_kv, c6.hd, cs6, c6.eps, kc6, vc6,
                                           wqk=wqk6, positions=pos6)[0],
            "qk_norm_rope": ops.prepare(ops.qk_norm_rope, qkv6, c6.n_q, c6.n_kv, c6.hd, cs6, c6.eps, wqk=wqk6,
                                        positions=pos6)[0],
            "store_kv": ops.prepare(ops.store_kv, qkv6, qoff, qoff + kw6, kw6, kc6, vc6, positions=pos6)[0],
        }
        bytes6 = {"add_rmsnorm": wl.bytes_add_rmsnorm(c6.T, c6.C),
                  "qk_norm_rope_kv": wl.bytes_qk_rope_kv(c6.T, c6.n_q, c6.n_kv, c6.hd),
                  "qk_norm_rope": wl.bytes_qk_rope(c6.T, c6.n_q, c6.n_kv, c6.hd),
                  "store_kv": wl.bytes_store_kv(c6.T, kw6)}
        # Floors of each op's byte pattern, over copies of its inputs: the residual add's two rows in and
        # two out (x in place), the q/k rows rewritten in place (with the KV store: k copied out as well,
        # v copied to its cache row), the k and v parts of each row split into the two caches.
        fl6 = FloorLib(torch.cuda.current_stream().cuda_stream)
        xf, df, cf = x6.clone(), d6.clone(), torch.empty_like(x6)
        qf, qf2, kf, vf = qkv6.clone(), qkv6.clone(), torch.empty_like(kc6), torch.empty_like(vc6)
        rs6, qk_w6, kvb = c6.qkv_stride * 2, (c6.n_q + c6.n_kv) * c6.hd * 2, kw6 * 2
        waves6 = 16 * torch.cuda.get_device_properties(dev).multi_processor_count
        floors6 = {"add_rmsnorm": [], "qk_norm_rope_kv": [], "qk_norm_rope": [], "store_kv": []}
        for items in (1, 4):
            for ntl, nts in ((1, 1), (0, 0)):
                name = f"floor_add2_i{items}_{'ntnt' if ntl else 'plpl'}"
                calls6[name] = fl6.add2(xf.data_ptr(), df.data_ptr(), cf.data_ptr(), c6.T * c6.C * 2, items, ntl, nts)
                floors6["add_rmsnorm"].append(name)
        calls6["floor_inplace_kv"] = fl6.inplace_kv(qf.data_ptr(), rs6, c6.T, qk_w6, kvb, kf.data_ptr(), vf.data_ptr(), kvb)
        floors6["qk_norm_rope_kv"].append("floor_inplace_kv")
        calls6["floor_inplace_plpl"] = fl6.inplace(qf2.data_ptr(), rs6, c6.T, qk_w6, 0, 0)
        calls6["floor_inplace_plpl_x64"] = fl6.inplace_x(qf2.data_ptr(), rs6, c6.T, qk_w6, 64)
        calls6["floor_inplace_rows_ntpl"] = fl6.inplace_rows(qf2.data_ptr(), rs6, c6.T, qk_w6, waves6, 1, 0)
        floors6["qk_norm_rope"] += ["floor_inplace_plpl", "floor_inplace_rows_ntpl", "floor_inplace_plpl_x64"]
        calls6["floor_split2"] = fl6.split2(qf2.data_ptr() + qoff * 2, rs6, kvb, kf.data_ptr(), vf.data_ptr(), kvb, c6.T)
        floors6["store_kv"].append("floor_split2")
        for fl_names in floors6.values():
            for f in fl_names:
                bytes6[f] = bytes6[next(k for k, v in floors6.items() if f in v)]
        run("qwen3_4b_fused", calls6, bytes6,
            "Qwen3-4B fused neighbours: residual add + RMSNorm [8192,2560]; q/k RoPE + KV store of an 8192-token "
            "sequence, beside the unfused q/k RoPE and KV store", floors=floors6)
        del xf, df, cf, qf, qf2, kf, vf

    # Qwen3-4B attention over the f16 KV cache (the reference's Attention kernel; cpu::attention), f32 q
    # and out as the adapter passes them: one decode token over 4096 and 32768 cached positions (bytes =
    # the k and v rows once + q + out: HBM-bound) and prefills of 2048 and 8192 tokens from position 0
    # (flops = 4 hd per (head, token, key): the q.k and p.v products).
    if want("qwen3_4b_attention"):
        c10 = wl.QWEN3_PREFILL
        H10, KV10, hd10 = c10.n_q, c10.n_kv, c10.hd
        kw10 = KV10 * hd10
        calls10, bytes10, flops10 = {}, {}, {}
        for name, T, pos0, _ in ATTENTION_CASES:
            q10 = wl.normal_f16((T, H10 * hd10), 0.0, 1.0, 101, dev).float()
            kc10 = wl.normal_f16((pos0 + T, kw10), 0.0, 1.0, 102, dev)
            vc10 = wl.normal_f16((pos0 + T, kw10), 0.0, 1.0, 103, dev)
            o10 = torch.empty_like(q10)
            calls10[name] = ops.prepare(ops.attention, q10, kc10, vc10, H10, KV10, hd10, pos0, out=o10)[0]
            calls10[name].keep = (q10, kc10, vc10, o10)
            bytes10[name] = (pos0 + T) * kw10 * 2 * 2 + 2 * T * H10 * hd10 * 4
            flops10[name] = 4 * hd10 * H10 * (T * pos0 + T * (T + 1) // 2)
        run("qwen3_4b_attention", calls10, bytes10,
            "Qwen3-4B attention (32 q / 8 kv heads x 128) over an f16 KV cache, f32 q and out: decode of one token "
            "over 4096 / 32768 cached positions, prefill of 2048 / 8192 tokens from position 0")
        for name, f in flops10.items():  # the kernel's products run on the f32 vector units
            op = out["qwen3_4b_attention"]["ops"][name]
            tf = f / (op["us"] * 1e-6) / 1e12
            op.update({"flops": f, "TFLOPs": round(tf, 2), "valu_f32_frac": round(tf / VALU_F32_PEAK_TFLOPS, 4)})
        del calls10

    # Load-time quantiser: the 151936 x 2048 tied table in f32 (1.24 GB) encoded on the device into each
    # weight format; bytes = the f32 rows read + the encoded rows written.
    if want("quantize_qwen3_1.7b_table"):
        c7 = wl.QUANT_GATHER
        src7 = wl.normal_f16((c7.vocab, c7.C), 0.0, 0.02, 31, dev).float()
        calls7, bytes7 = {}, {}
        for fmt, name in ((ops.FMT_F16, "quantize_fp16"), (ops.FMT_FP8, "quantize_fp8"), (ops.FMT_FP4, "quantize_fp4")):
            run7, (tab7, _) = ops.prepare(ops.quantize, src7, fmt)
            calls7[name] = run7
            run7.table = tab7  # keep the output alive with its call
            bytes7[name] = c7.vocab * c7.C * 4 + tab7.numel()
        run("quantize_qwen3_1.7b_table", calls7, bytes7,
            "quantizeMatrix on the device: 151936 x 2048 f32 table -> F16 / FP8 / FP4 rows")
        del src7, calls7

    # Granite-4.0-H-style norms and SwiGLU
    if want("granite_4.0h_norms"):
        c5 = wl.GRANITE_NORMS
        x5 = wl.normal_f16((c5.T, c5.C), 0.0, 1.0, 51, dev)
        w5 = wl.weight_f32(c5.C, 1.0, 0.05, 52, dev)
        y5 = torch.empty_like(x5)
        ya = wl.normal_f16((c5.T, c5.D), 0.0, 1.0, 53, dev)
        za = wl.normal_f16((c5.T, c5.D), 0.0, 1.0, 54, dev)
        wg = wl.weight_f32(c5.D, 1.0, 0.05, 55, dev)
        og = torch.empty_like(ya)
        h5 = wl.normal_f16((c5.T, 2 * c5.I), 0.0, 1.0, 56, dev)
        o5 = torch.empty((c5.T, c5.I), dtype=torch.float16, device=dev)
        calls5 = {
            "rmsnorm": ops.prepare(ops.rms_norm, x5, w5, c5.eps, out=y5)[0],
            "gated_rmsnorm": ops.prepare(ops.gated_rms_norm, ya, za, wg, c5.groups, c5.eps, out=og)[0],
            "swiglu": ops.prepare(ops.silu_mul, h5, out=o5)[0],
        }
        bytes5 = {"rmsnorm": wl.bytes_rmsnorm(c5.T, c5.C), "gated_rmsnorm": wl.bytes_gated(c5.T, c5.D),
                  "swiglu": wl.bytes_swiglu(c5.T, c5.I)}
        # Floors of each op's byte pattern, reading the op's own inputs: copies of the RMSNorm's rows, the
        # gated norm's y and z rows into one output row, SwiGLU's two halves of each row into one.
        fl5 = FloorLib(torch.cuda.current_stream().cuda_stream)
        y5f, og5f, o5f = torch.empty_like(y5), torch.empty_like(og), torch.empty_like(o5)
        floors5 = {"rmsnorm": [], "gated_rmsnorm": ["floor_gate"], "swiglu": ["floor_rows2_ntpl"]}
        for items in (1, 4):
            for ntl, nts in ((1, 1), (0, 0)):
                name = f"floor_copy_i{items}_{'ntnt' if ntl else 'plpl'}"
                calls5[name] = fl5.copy(x5.data_ptr(), y5f.data_ptr(), c5.T * c5.C * 2, items, ntl, nts)
                floors5["rmsnorm"].append(name)
                bytes5[name] = bytes5["rmsnorm"]
        calls5["floor_copy_i1_plpl_x128"] = fl5.copy_x(x5.data_ptr(), y5f.data_ptr(), c5.T * c5.C * 2, 0, 0, 128)
        floors5["rmsnorm"].append("floor_copy_i1_plpl_x128")
        bytes5["floor_copy_i1_plpl_x128"] = bytes5["rmsnorm"]
        calls5["floor_gate"] = fl5.gate(ya.data_ptr(), c5.D * 2, za.data_ptr(), c5.D * 2, og5f.data_ptr(), c5.D * 2,
                                        c5.D * 2, c5.T)
        bytes5["floor_gate"] = bytes5["gated_rmsnorm"]
        calls5["floor_rows2_ntpl"] = fl5.rows2(h5.data_ptr(), 2 * c5.I * 2, o5f.data_ptr(), c5.I * 2, c5.T, c5.I * 2, 1, 0)
        calls5["floor_rows2_ntpl_x128"] = fl5.rows2_x(h5.data_ptr(), 2 * c5.I * 2, o5f.data_ptr(), c5.I * 2, c5.T, c5.I * 2, 128)
        floors5["swiglu"].append("floor_rows2_ntpl_x128")
        bytes5["floor_rows2_ntpl"] = bytes5["floor_rows2_ntpl_x128"] = bytes5["swiglu"]
        run("granite_4.0h_norms", calls5, bytes5,
            "Granite-4.0-H: 16384 tokens, RMSNorm 1536, gated RMSNorm y*silu(z) 3072, SwiGLU I=4096", floors=floors5)
        del y5f, og5f, o5f

    # Qwen3-4B decode step (T = 1): the four weight matmuls in each weight format, f16 activations,
    # f32 outputs; bytes = the weight rows once + activations + outputs.
    # Qwen3-4B decode steps of 1, 4, 16 and 24 sequences: the layer's four weight matmuls,
    # weight-bandwidth bound.
    # The _f32 forms take f32 activations, the type the reference's ComputeBackend (the adapter) passes.
    for label8, c8, x32 in (("qwen3_4b_decode_matmul", wl.QWEN3_DECODE_MATMUL, False),
                            ("qwen3_4b_decode4_matmul", wl.QWEN3_DECODE4_MATMUL, False),
                            ("qwen3_4b_decode16_matmul", wl.QWEN3_DECODE16_MATMUL, False),
                            ("qwen3_4b_decode24_matmul", wl.QWEN3_DECODE24_MATMUL, False),
                            ("qwen3_4b_decode_matmul_f32", wl.QWEN3_DECODE_MATMUL, True),
                            ("qwen3_4b_decode16_matmul_f32", wl.QWEN3_DECODE16_MATMUL, True)):
        if not want(label8):
            continue
        calls8, bytes8 = {}, {}
        for pname, N, K in c8.projections:
            wsrc = wl.normal_f16((N, K), 0.0, 0.02, 81, dev).float()
            x8 = wl.normal_f16((c8.T, K), 0.0, 1.0, 82, dev)
            if x32:
                x8 = x8.float()
            y8 = torch.empty((c8.T, N), dtype=torch.float32, device=dev)
            for fmt, fname in ((ops.FMT_F16, "f16"), (ops.FMT_FP8, "fp8"), (ops.FMT_FP4, "fp4")):
                tab8, _ = ops.quantize(wsrc, fmt)
                name = f"{pname}_{fname}"
                calls8[name] = ops.prepare(ops.matmul, x8, tab8, fmt, K, out=y8)[0]
                calls8[name].table = tab8
                bytes8[name] = wl.bytes_matmul(c8.T, K, N, tab8.shape[1], x_bytes=4 if x32 else 2)
            del wsrc
        run(label8, calls8, bytes8,
            f"Qwen3-4B decode step, T={c8.T}: q/k/v [6144,2560], o [2560,4096], gate/up [19456,2560], down [2560,9728] "
            f"weight matmuls in F16 / FP8 / FP4 rows, {'f32' if x32 else 'f16'} activations, f32 outputs")
        del calls8

    # Qwen3-4B prefill (T = 8192): the same four weight matmuls, MFMA-bound; flops = 2 T N K.
    if want("qwen3_4b_prefill_matmul"):
        c9 = wl.QWEN3_PREFILL_MATMUL
        calls9, bytes9, flops9, lib9 = {}, {}, {}, {}
        for pname, N, K in c9.projections:
            wsrc = wl.normal_f16((N, K), 0.0, 0.02, 91, dev).float()
            x9 = wl.normal_f16((c9.T, K), 0.0, 1.0, 92, dev)
            y9 = torch.empty((c9.T, N), dtype=torch.float32, device=dev)
            # The vendor library on the same F16 product (torch -> hipBLASLt), with f16 output and with
            # f32 output (this path's own): a reference point for the MFMA kernel, not part of the path.
            w16, y16 = wsrc.half(), torch.empty((c9.T, N), dtype=torch.float16, device=dev)
            lib9[f"{pname}_f16_out16"] = (lambda x=x9, w=w16, y=y16: torch.matmul(x, w.t(), out=y))
            lib9[f"{pname}_f16"] = (lambda x=x9, w=w16: torch.mm(x, w.t(), out_dtype=torch.float32))
            for fmt, fname in ((ops.FMT_F16, "f16"), (ops.FMT_FP8, "fp8"), (ops.FMT_FP4, "fp4")):
                tab9, _ = ops.quantize(wsrc, fmt)
                name = f"{pname}_{fname}"
                calls9[name] = ops.prepare(ops.matmul, x9, tab9, fmt, K, out=y9)[0]
                calls9[name].table = tab9
                bytes9[name] = wl.bytes_matmul(c9.T, K, N, tab9.shape[1])
                flops9[name] = 2 * c9.T * N * K
                if fmt == ops.FMT_F16:  # the library's product exactly: f16 output
                    ours16 = torch.empty((c9.T, N), dtype=torch.float16, device=dev)
                    calls9[f"{name}_out16"] = ops.prepare(ops.matmul, x9, tab9, fmt, K, out=ours16)[0]
                    calls9[f"{name}_out16"].keep = (tab9, ours16)
                    bytes9[f"{name}_out16"] = wl.bytes_matmul(c9.T, K, N, tab9.shape[1], y_bytes=2)
                    flops9[f"{name}_out16"] = flops9[name]
                    # The same product on this library's own MFMA kernels (the context's hipBLASLt
                    # dispatch switched off around the call).
                    ctx9 = ops.context(dev.index or 0)
                    run_lib = calls9[name]

                    def own(run=run_lib, c=ctx9):
                        c.set_matmul_library(False)
                        try:
                            run()
                        finally:
                            c.set_matmul_library(True)
                    calls9[f"{name}_own"], bytes9[f"{name}_own"], flops9[f"{name}_own"] = own, bytes9[name], flops9[name]
            del wsrc
        run("qwen3_4b_prefill_matmul", calls9, bytes9,
            "Qwen3-4B prefill, T=8192: q/k/v [6144,2560], o [2560,4096], gate/up [19456,2560], down [2560,9728] "
            "weight matmuls in F16 / FP8 / FP4 rows, f16 activations, f32 outputs", flops9)
        lib_ops, _ = time_ops(lib9, bytes9, list(lib9), args.steps, args.warmup, flush,
                              HipTimer(torch.cuda.current_stream().cuda_stream))
        ops9 = out["qwen3_4b_prefill_matmul"]["ops"]
        for n, v in lib_ops.items():
            tf = flops9[n] / (v["us"] * 1e-6) / 1e12
            kind = "f16" if n.endswith("_out16") else "f32"
            for m in (n, f"{n}_own"):  # the op as shipped, and on the own kernels
                if m in ops9:
                    ops9[m].update({"library_us": v["us"], "library_TFLOPs": round(tf, 1),
                                    "library": f"torch f16 x f16 -> {kind} (hipBLASLt)",
                                    "vs_library": round(v["us"] / ops9[m]["us"], 4)})
        del calls9, lib9

    if not args.no_cpu:
        del flush
        torch.cuda.synchronize()
        leg = CpuLeg()
        add_cpu_jobs(leg, want)
        leg.run(out)
    return out


def _fit(points):
    """Least-squares time = fixed + bytes / rate over (bytes, us) points: (fixed us, rate GB/s)."""
    n = len(points)
    mx = sum(b for b, _ in points) / n
    my = sum(t for _, t in points) / n
    sxx = sum((b - mx) ** 2 for b, _ in points)
    slope = sum((b - mx) * (t - my) for b, t in points) / sxx  # us per byte
    return round(my - slope * mx, 3), round(1e-3 / slope, 1)


def stream_floor(args, flush, time_ops):
    """What moving the ops' bytes costs with nothing else to do, timed like the ops (same flush and
    events): an empty kernel; 16-byte-per-lane copies with the byte patterns of the Qwen3-4B prefill
    ops (RMSNorm: read 42 MB / write 42 MB; q/k RoPE: 84 / 84; SwiGLU: two 159 MB streams in, one
    out), and the same bytes in SwiGLU's and the q/k RoPE's own row layouts; the HIP runtime's own
    device-to-device copies (hipMemcpyAsync, hipMemcpy2DAsync, torch's copy_) of the same bytes; a
    read-only sweep; the RMSNorm at 4096-32768 rows of 2560 beside copies of the same bytes, with the
    straight-line fits time = fixed + bytes / rate of both; the RMSNorm and the read sweep after 1, 2
    and 4 GiB flushes; and each headline op (and its floor) with a 1 GiB read sweep after it inside the
    event pair, beside the sweep alone -- the difference is the op plus any write-back of its output
    that the op's own end event does not wait for."""
    import torch

    from nekochat_amd import ops
    from nekochat_amd import workloads as wl

    dev = torch.device("cuda:0")
    fl = FloorLib(torch.cuda.current_stream().cuda_stream)

    cfg = wl.QWEN3_PREFILL
    big = 2 * cfg.T * cfg.I * 2  # bytes of the SwiGLU input rows, the largest stream
    # Random bits in every source (and in the in-place buffer): with constant or zero data the copies
    # run measurably faster than they do on activations, so they would understate the floor.
    gen = torch.Generator(device=dev)
    gen.manual_seed(12345)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (big // 4,), dtype=torch.int32, device=dev, generator=gen)
    dst = torch.randint(-2 ** 31, 2 ** 31 - 1, (big // 4,), dtype=torch.int32, device=dev, generator=gen)
    sink = torch.zeros(1024, dtype=torch.float32, device=dev)
    a_ptr, d_ptr = src.data_ptr(), dst.data_ptr()
    calls, nbytes = {}, {}
    calls["empty_1wg"], nbytes["empty_1wg"] = fl.empty(1), 0
    calls["empty_8192wg"], nbytes["empty_8192wg"] = fl.empty(8192), 0
    half = cfg.T * cfg.C * 2
    patterns = {"rmsnorm": half, "qk_norm_rope": 2 * cfg.T * (cfg.n_q + cfg.n_kv) * cfg.hd}
    for label, each in patterns.items():  # read `each` bytes, write `each` bytes
        for items in (1, 4):
            for ntl, nts in ((1, 1), (1, 0), (0, 0)):
                name = f"copy_{label}_i{items}_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}"
                calls[name] = fl.copy(a_ptr, d_ptr, each, items, ntl, nts)
                nbytes[name] = 2 * each
        # one chunk per lane with the workgroups' data in runs of 64 / 128 / 256 per XCD
        for run_ in (64, 128, 256):
            for nt in (1, 0):
                name = f"copy_{label}_i1_{'ntnt' if nt else 'plpl'}_x{run_}"
                calls[name] = fl.copy_x(a_ptr, d_ptr, each, nt, nt, run_)
                nbytes[name] = 2 * each
        # the runtime's copy of the same bytes, and torch's copy_ (which calls it)
        calls[f"hipMemcpyAsync_{label}"], nbytes[f"hipMemcpyAsync_{label}"] = fl.memcpy(d_ptr, a_ptr, each), 2 * each
        sv, dv = src[:each // 4], dst[:each // 4]
        calls[f"torch_copy__{label}"], nbytes[f"torch_copy__{label}"] = (lambda d=dv, s=sv: d.copy_(s)), 2 * each
    gi = cfg.T * cfg.I * 2  # SwiGLU: gate and up streams of T x I halves in, T x I out
    for ntl, nts in ((1, 1), (1, 0), (0, 0)):
        name = f"copy2_swiglu_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}"
        calls[name] = fl.copy2(a_ptr, a_ptr + gi, d_ptr, gi, ntl, nts)
        nbytes[name] = 3 * gi
    # The runtime's copies cannot read two bytes for each one written: the gate halves of the
    # [T, 2I] rows copied out (159 + 159 MB, 2D), and a flat copy of the op's total (239 + 239 MB).
    calls["hipMemcpy2DAsync_swiglu_gate"] = fl.memcpy2d(d_ptr, gi // cfg.T, a_ptr, 2 * gi // cfg.T, gi // cfg.T, cfg.T)
    nbytes["hipMemcpy2DAsync_swiglu_gate"] = 2 * gi
    calls["hipMemcpyAsync_swiglu_same_total"] = fl.memcpy(d_ptr, a_ptr, 3 * gi // 2)
    nbytes["hipMemcpyAsync_swiglu_same_total"] = 3 * gi
    # The same bytes in the ops' own layouts: SwiGLU's gate and up halves of one [T, 2I] row into a
    # [T, I] row; the q/k RoPE's in-place rewrite of the first (n_q + n_kv) hd halves of each qkv row.
    for ntl, nts in ((1, 0), (1, 1), (0, 0)):
        name = f"rows2_swiglu_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}"
        calls[name] = fl.rows2(a_ptr, 2 * gi // cfg.T, d_ptr, gi // cfg.T, cfg.T, gi // cfg.T, ntl, nts)
        nbytes[name] = 3 * gi
    for run_ in (64, 128, 256):  # SwiGLU's layout and cache policy in XCD order
        name = f"rows2_swiglu_ntpl_x{run_}"
        calls[name] = fl.rows2_x(a_ptr, 2 * gi // cfg.T, d_ptr, gi // cfg.T, cfg.T, gi // cfg.T, run_)
        nbytes[name] = 3 * gi
    # The same SwiGLU-layout stream over constant input (every output line zero): how much cheaper
    # uniform data is, the reason the sources above are random.
    # Its output goes to a buffer of its own: written into the shared destination, it left constant data
    # there that the in-place floors after it then rewrote faster than random bits.
    ones = torch.ones(big // 4, dtype=torch.float32, device=dev)
    const_out = torch.empty(gi // 4, dtype=torch.int32, device=dev)
    calls["rows2_swiglu_ntpl_constdata"] = fl.rows2(ones.data_ptr(), 2 * gi // cfg.T, const_out.data_ptr(), gi // cfg.T,
                                                    cfg.T, gi // cfg.T, 1, 0)
    nbytes["rows2_swiglu_ntpl_constdata"] = 3 * gi
    # The one-round shape (every row of a wave loaded before its stores; two rows per wave at 8192
    # rows), with and without a workgroup barrier between the reads and the writes: the RMSNorm's bytes
    # copied, the q/k rows rewritten in place.
    qk_w = (cfg.n_q + cfg.n_kv) * cfg.hd * 2
    for sync in (0, 1):
        tag = "_sync" if sync else ""
        calls[f"rows_up_rmsnorm_r2{tag}"] = fl.rows_up(a_ptr, cfg.C * 2, d_ptr, cfg.C * 2, cfg.T, 2, cfg.C * 2 // 1024, sync)
        nbytes[f"rows_up_rmsnorm_r2{tag}"] = 2 * half
        calls[f"rows_up_qk_inplace_r2{tag}"] = fl.rows_up(d_ptr, cfg.qkv_stride * 2, d_ptr, cfg.qkv_stride * 2, cfg.T, 2,
                                                          qk_w // 1024, sync)
        nbytes[f"rows_up_qk_inplace_r2{tag}"] = 2 * cfg.T * qk_w
    for ntl, nts in ((0, 0), (1, 0), (1, 1), (0, 1)):
        name = f"inplace_qk_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}"
        calls[name] = fl.inplace(d_ptr, cfg.qkv_stride * 2, cfg.T, qk_w, ntl, nts)
        nbytes[name] = 2 * cfg.T * qk_w
    for run_ in (64, 128, 256):
        name = f"inplace_qk_plpl_x{run_}"
        calls[name] = fl.inplace_x(d_ptr, cfg.qkv_stride * 2, cfg.T, qk_w, run_)
        nbytes[name] = 2 * cfg.T * qk_w
    # The op itself on the headline's inputs, and the same rewrite of its own qkv buffer in the q/k
    # kernel's schedule: whole rows per wave, wave w taking rows w, w + nw, ..., at the kernel's
    # occupancy of four waves per SIMD (its load policy first), all timed in the same rounds.
    qk_in = wl.qwen3_prefill_inputs(cfg, dev)
    calls["qk_norm_rope_op"] = ops.prepare(ops.qk_norm_rope, qk_in["qkv"], cfg.n_q, cfg.n_kv, cfg.hd, qk_in["cs"], cfg.eps,
                                           wqk=qk_in["wqk"], positions=qk_in["positions"])[0]
    nbytes["qk_norm_rope_op"] = wl.bytes_qk_rope(cfg.T, cfg.n_q, cfg.n_kv, cfg.hd)
    # The RMSNorm's bytes copied from its own input rows (f16 activations) instead of random bits.
    x_own = qk_in["x"]
    x_dst = torch.empty_like(x_own)
    for items, ntl, nts in ((1, 1, 1), (4, 0, 0)):
        name = f"copy_rmsnorm_i{items}_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}_owndata"
        calls[name], nbytes[name] = fl.copy(x_own.data_ptr(), x_dst.data_ptr(), half, items, ntl, nts), 2 * half
    calls["rows_up_rmsnorm_r2_owndata"] = fl.rows_up(x_own.data_ptr(), cfg.C * 2, x_dst.data_ptr(), cfg.C * 2, cfg.T, 2,
                                                     cfg.C * 2 // 1024, 0)
    nbytes["rows_up_rmsnorm_r2_owndata"] = 2 * half
    waves = 16 * torch.cuda.get_device_properties(dev).multi_processor_count
    for ntl, nts in ((1, 0), (0, 0)):
        name = f"inplace_qk_rows_{'nt' if ntl else 'pl'}{'nt' if nts else 'pl'}"
        calls[name] = fl.inplace_rows(qk_in["qkv"].data_ptr(), cfg.qkv_stride * 2, cfg.T, qk_w, waves, ntl, nts)
        nbytes[name] = 2 * cfg.T * qk_w
    # (and the flat rewrite over that buffer too, and the runtime's 2D copy of those bytes elsewhere)
    calls["inplace_qk_plpl_opbuf"] = fl.inplace(qk_in["qkv"].data_ptr(), cfg.qkv_stride * 2, cfg.T, qk_w, 0, 0)
    nbytes["inplace_qk_plpl_opbuf"] = 2 * cfg.T * qk_w
    qk_copy = torch.empty_like(qk_in["qkv"])
    calls["hipMemcpy2DAsync_qk"] = fl.memcpy2d(qk_copy.data_ptr(), cfg.qkv_stride * 2, qk_in["qkv"].data_ptr(),
                                               cfg.qkv_stride * 2, qk_w, cfg.T)
    nbytes["hipMemcpy2DAsync_qk"] = 2 * cfg.T * qk_w
    calls["read_rmsnorm_in"], nbytes["read_rmsnorm_in"] = fl.read(a_ptr, half, sink.data_ptr()), half
    # RMSNorm [rows, 2560] at four row counts, and copies of the same bytes.
    w = wl.weight_f32(cfg.C, 1.0, 0.05, 2, dev)
    sweep = (4096, 8192, 16384, 32768)
    norm_io = {}
    for rows in sweep:
        x = wl.normal_f16((rows, cfg.C), 0.0, 1.0, 1, dev)
        y = torch.empty_like(x)
        norm_io[rows] = (x, y)
        calls[f"rmsnorm_rows{rows}"] = ops.prepare(ops.rms_norm, x, w, cfg.eps, out=y)[0]
        nbytes[f"rmsnorm_rows{rows}"] = wl.bytes_rmsnorm(rows, cfg.C)
        calls[f"copy_rows{rows}"] = fl.copy(a_ptr, d_ptr, rows * cfg.C * 2, 1, 1, 1)
        nbytes[f"copy_rows{rows}"] = 2 * rows * cfg.C * 2
    # Flush size: the RMSNorm, its copy and the read sweep after 1, 2 and 4 GiB read sweeps (the
    # default rounds above use 1 GiB).
    flushes = {}
    big_flush = {g: torch.ones(g * (256 << 20), dtype=torch.float32, device=dev) for g in (2, 4)}
    big_flush[1] = flush
    for g in (1, 2, 4):
        for base in ("rmsnorm_rows8192", "copy_rows8192", "read_rmsnorm_in"):
            name = f"{base}_flush{g}gib"
            calls[name], nbytes[name], flushes[name] = calls[base], nbytes[base], big_flush[g]
    # Trailing write-back: each headline op (and the floors of its pattern) followed by a 1 GiB read
    # sweep inside the same event pair, and the sweep alone after the same flush.
    tails = {}
    trail = torch.ones(256 << 20, dtype=torch.float32, device=dev)  # not the flush buffer: no hits in it

    def sweep_once():
        trail.sum()

    h_in = qk_in["h"]
    g_out = torch.empty((cfg.T, cfg.I), dtype=torch.float16, device=dev)
    xn = torch.empty_like(qk_in["x"])
    trailed = {
        "rmsnorm_op": (ops.prepare(ops.rms_norm, qk_in["x"], qk_in["w_in"], cfg.eps, out=xn)[0],
                       wl.bytes_rmsnorm(cfg.T, cfg.C)),
        "copy_rmsnorm_i1_ntnt": (calls["copy_rmsnorm_i1_ntnt"], nbytes["copy_rmsnorm_i1_ntnt"]),
        "hipMemcpyAsync_rmsnorm": (calls["hipMemcpyAsync_rmsnorm"], nbytes["hipMemcpyAsync_rmsnorm"]),
        "qk_norm_rope_op": (calls["qk_norm_rope_op"], nbytes["qk_norm_rope_op"]),
        "inplace_qk_rows_ntpl": (calls["inplace_qk_rows_ntpl"], nbytes["inplace_qk_rows_ntpl"]),
        "swiglu_op": (ops.prepare(ops.silu_mul, h_in, out=g_out)[0], wl.bytes_swiglu(cfg.T, cfg.I)),
        "rows2_swiglu_ntpl": (calls["rows2_swiglu_ntpl"], nbytes["rows2_swiglu_ntpl"]),
    }
    calls["sweep1gib_alone"], nbytes["sweep1gib_alone"] = sweep_once, 1 << 30
    for base, (fn, nb) in trailed.items():
        name = f"{base}+sweep1gib"
        calls[name], nbytes[name], tails[name] = fn, nb, sweep_once
        if base not in calls:
            calls[base], nbytes[base] = fn, nb
    timer = HipTimer(torch.cuda.current_stream().cuda_stream)
    per_op, _ = time_ops(calls, nbytes, list(calls), args.steps, args.warmup, flush, timer, flushes=flushes,
                         tails=tails)
    torch.cuda.synchronize()
    fits = {kind: _fit([(nbytes[f"{kind}_rows{r}"], per_op[f"{kind}_rows{r}"]["us"]) for r in sweep])
            for kind in ("rmsnorm", "copy")}
    alone = per_op["sweep1gib_alone"]["us"]
    writeback = {base: {"op_us": per_op[base]["us"], "op_plus_sweep_minus_sweep_us": round(per_op[f"{base}+sweep1gib"]["us"] - alone, 3)}
                 for base in trailed}
    for v in writeback.values():
        v["hidden_us"] = round(v["op_plus_sweep_minus_sweep_us"] - v["op_us"], 3)
    flush_size = {base: {f"{g}GiB": per_op[f"{base}_flush{g}gib"]["us"] for g in (1, 2, 4)}
                  for base in ("rmsnorm_rows8192", "copy_rows8192", "read_rmsnorm_in")}
    del big_flush
    return {"workload": "streaming floor: empty kernels, 16-byte copies with the Qwen3-4B prefill ops' byte patterns, "
                        "the runtime's device-to-device copies of the same bytes, RMSNorm rows sweep at hidden 2560 "
                        "beside copies of the same bytes, flush-size and trailing write-back checks",
            "ops": per_op,
            "fit_us_plus_bytes_per_rate": {k: {"fixed_us": v[0], "GBps": v[1]} for k, v in fits.items()},
            "flush_size_us": flush_size,
            "trailing_writeback": {"sweep_alone_us": alone, "ops": writeback}}


def cpu_baseline(cfg, rows=None, reps=5):
    """The reference's CPU path for the layer's four ops (its compiled cpu::rmsNorm, the Qwen3 q/k loop
    of rmsNorm + rope, cpu::siluMul on f32 activations, as its CPU forward pass holds them) on one
    pinned core over `rows` tokens of the same workload (default: all of them, ~0.2 s per layer),
    scaled to the full layer; the oracle's f32 restatement when oracle/_ref is not built."""
    import numpy as np

    from nekochat_amd import workloads as wl
    from oracle import oracle as O

    rows = cfg.T if rows is None else rows
    x = _f32((rows, cfg.C), 0.0, 1.0, 1)
    w = wl.weight_f32(cfg.C, 1.0, 0.05, 2, "cpu").numpy()
    qkv = _f32((rows, cfg.qkv_stride), 0.0, 1.0, 4)
    wqk = wl.weight_f32(2 * cfg.hd, 1.0, 0.05, 5, "cpu").numpy()
    wq, wk = wqk[:cfg.hd].copy(), wqk[cfg.hd:].copy()
    pos = (np.arange(rows) % cfg.seq).astype(np.int32)
    cs = O.rope_table(cfg.theta, cfg.hd, cfg.seq)
    h = _f32((rows, 2 * cfg.I), 0.0, 1.0, 6)
    y = np.empty_like(x)
    g = np.empty((rows, cfg.I), np.float32)
    P = O._ptr
    if O.ref_available():
        R = O.ref()
        kind = "reference"
        run = {
            "rmsnorm": lambda: R.ref_rmsnorm(P(x), P(y), P(w), rows, cfg.C, cfg.eps),
            "qk_norm_rope": lambda: R.ref_qk_norm_rope(P(qkv), cfg.qkv_stride, rows, cfg.n_q, cfg.n_kv, cfg.hd,
                                                       P(pos), P(wq), P(wk), P(cs), cfg.eps),
            "swiglu": lambda: R.ref_silu_mul(P(h), P(g), rows, cfg.I),
        }
    else:
        kind = "port"
        L = O.lib()
        run = {
            "rmsnorm": lambda: L.oracle_rmsnorm(P(x), P(y), P(w), rows, cfg.C, cfg.eps),
            "qk_norm_rope": lambda: L.oracle_qk_norm_rope_f32(P(qkv), cfg.qkv_stride, rows, cfg.n_q, cfg.n_kv,
                                                              cfg.hd, 0, P(pos), P(wqk), P(cs), cfg.seq, cfg.eps),
            "swiglu": lambda: L.oracle_silu_mul(P(h), P(g), rows, cfg.I),
        }
    mask = _pin_one_core()
    t = {}
    for name, fn in run.items():
        fn()
        samples = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            samples.append(time.perf_counter() - t0)
        t[name] = statistics.median(samples) * cfg.T / rows  # seconds for the full 8192 rows
    _unpin(mask)
    layer_s = 2 * t["rmsnorm"] + t["qk_norm_rope"] + t["swiglu"]
    total_bytes = sum(cfg.op_bytes().values())
    return {
        "value": round(total_bytes / layer_s / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
        "us_per_layer": round(layer_s * 1e6, 1),
        "per_op_us": {k: round(v * 1e6, 1) for k, v in t.items()},
        "sample": (f"the full {cfg.T}-token layer" if rows == cfg.T else f"{rows} of {cfg.T} tokens, scaled to the full layer")
                  + f" per op (median of {reps}); 1 pinned core of {os.cpu_count()}; g++ -O3 portable x86-64 build; "
                  "f32 activations",
    }


# The dominant kernel's sources: its file, the device helpers it uses, and the build flags.
TRAFFIC_SOURCES = ("nekochat_amd/csrc/act.hip", "nekochat_amd/csrc/device.h", "nekochat_amd/csrc/Makefile")


def sources_sha256(paths=TRAFFIC_SOURCES) -> str:
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        h.update(rel.encode() + b"\0")
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def traffic_from_profiles():
    """(bytes, note): the dominant kernel's per-launch HBM bytes from rocprofv3 FETCH_SIZE / WRITE_SIZE
    (profiles/), when those counters were taken on the kernel sources as they are now (the profile
    records their sha256); otherwise (None, why)."""
    path = os.path.join(ROOT, "profiles", "swiglu_qwen3_4b_prefill_traffic.json")
    if not os.path.exists(path):
        return None, "no counter profile recorded"
    with open(path) as f:
        rec = json.load(f)
    have = sources_sha256(rec.get("sources", TRAFFIC_SOURCES))
    if rec.get("sources_sha256") != have:
        return None, (f"counter profile taken on other {rec.get('kernel', 'kernel')} sources (sha256 "
                      f"{str(rec.get('sources_sha256'))[:12]} vs {have[:12]} now): not quoted")
    return rec["traffic_bytes_per_launch"], (f"rocprofv3 FETCH_SIZE + WRITE_SIZE of {rec['kernel']}, calibrated on "
                                             f"a device copy; sources sha256 {have[:12]} = the current sources'")


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: measures one GPU; the ops are per-row and shard by tokens with no "
              "communication, so N > 1 is not run here.", file=sys.stderr)
        sys.exit(2)
    if args.all:
        print(json.dumps({"metric": METRIC, "unit": "GB/s", "data": "synthetic", "configs": all_configs(args)}),
              flush=True)
        return
    cfg, per_op, wall, layer, floors = gpu_bench(args)
    sum_us = sum(v["us"] for v in per_op.values())
    total_bytes = sum(v["bytes"] for v in per_op.values())
    # The step: the layer's ops back-to-back after one flush, one event pair (median over steps);
    # with --only, the one op.
    total_us = statistics.median(layer) * 1e3 if layer else sum_us
    value = total_bytes / (total_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_us / 1e3, 5),
        "wall_ms_per_step": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Qwen3-4B prefill layer, non-GEMM ops: 2x RMSNorm [8192,2560] + q/k RMSNorm+NeoX RoPE "
                        "(32q+8kv x 128) + SwiGLU [8192,9728]; fp16 I/O, f32 math, f64 norm sums",
            "tokens": cfg.T, "hidden": cfg.C, "heads": [cfg.n_q, cfg.n_kv], "head_dim": cfg.hd,
            "intermediate": cfg.I, "io_dtype": "f16", "cache_flush": not args.no_flush,
        },
        "us_per_layer": round(total_us, 3),
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "us_per_layer_sum_of_ops": round(sum_us, 3),
        "ops": per_op,
    }
    if layer:
        line["layer_mean_us"] = round(statistics.fmean(layer) * 1e3, 3)
    if floors:
        # Each op beside the fastest byte-moving floor of its own pattern, timed in the same run.
        for op, d in per_op.items():
            b = floors["best"][op]
            d["floor_us"], d["floor_kind"] = b["us"], b["kind"]
            d["over_floor"] = round(d["us"] / b["us"] - 1, 4)
        line["floors"] = {"candidates_us": floors["candidates_us"], "layer_floor_us": floors["layer_step_us"],
                          "layer_over_floor": round(total_us / floors["layer_step_us"] - 1, 4)}
    if not args.only or args.only == DOMINANT:
        d = per_op[DOMINANT]
        achieved = d["bytes"] / (d["mean_us"] * 1e-6) / 1e9
        traffic, note = traffic_from_profiles()
        line["roofline"] = {"bound": "hbm", "kernel": DOMINANT, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                            "traffic_source": note}
    if not args.no_cpu and not args.only:
        line["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
