"""Benchmark: Gemma-3-1B-architecture Q8_0 batch-1 greedy decode after a
2048-token context, on one MI355X, through the C-ABI.

A "step" is one decode token: forward pass over 26 layers + tied LM head +
greedy selection, with the token read back to the host (one gg_step call, as
the reference's per-token loop does). Weights are seeded random-init Q8_0 of
the 1B architecture (no checkpoint is available offline); the KV cache holds
2048 positions from a batched prefill of seeded ids before timing (--ctx
changes the context, e.g. --ctx 32760 for the long-context case).

Prints one JSON line. `roofline` covers the dominant kernel: a second engine
runs the same decode steps with its kernels launched directly, and HIP events
around that kernel's launch give its mean duration. `prefill` reports the
TTFT of the batched prefill and its matrix-core utilisation; `cpu_baseline`
times the C oracle (a CPU restatement of the reference pipeline) on a bounded
sample of the same decode steps.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "webgpu-gemma_amd")]

import numpy as np  # noqa: E402

from gemma_amd import capi, synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
METRIC = "Gemma-3-1B Q8_0 bs1 decode tok/s @ctx2k; HBM GB/s as % of peak; prefill TTFT"


def step_bytes(shape, pos: int) -> int:
    """Algorithmic HBM bytes of one decode token at position `pos`: Q8_0
    weights at 34 B / 32, f32 norm weights, the f32 KV span each layer
    attends to, the KV row written, and the 1 MiB logits written + read."""
    H, L = shape.hidden, shape.layers
    w = shape.q8_bytes()
    norms = L * 4 * (4 * H + 2 * shape.head_dim) + 4 * H
    kv = 0
    for l in range(L):
        swa = (l % shape.swa_period) < shape.swa_period - 1
        span = pos + 1 if not (swa and shape.window) else min(shape.window, pos + 1)
        kv += span * 2 * shape.kv_dim * 4
    kv_write = L * 2 * shape.kv_dim * 4
    logits = 2 * shape.vocab * 4
    return w + norms + kv + kv_write + logits


def kernel_bytes(shape, kind: str, pos: int) -> int:
    """Algorithmic bytes of one launch of the probed kernel (weights at
    34 B / 32 + f32 input and output vectors)."""
    H, I, V, Q = shape.hidden, shape.inter, shape.vocab, shape.q_dim
    nqkv = Q + 2 * shape.kv_dim
    q8 = lambda rows, k: rows * k // 32 * 34  # noqa: E731
    if kind == "qkv":
        return q8(nqkv, H) + 4 * H + 4 * nqkv
    if kind == "o":
        return q8(H, Q) + 4 * Q + 4 * H
    if kind == "gate_up":
        return q8(2 * I, H) + 4 * H + 4 * I
    if kind == "down":
        return q8(H, I) + 4 * I + 4 * H
    if kind == "lm_head":
        return q8(V, H) + 4 * H + 4 * V
    raise ValueError(kind)


def prefill_flops(shape, m: int):
    """Algorithmic FLOPs of an m-token prefill: (GEMMs, attention) -- the GEMMs
    2 * m * layer weights, causal attention QK and PV over the span each layer
    attends to."""
    per_layer = shape.hidden * (shape.q_dim + 2 * shape.kv_dim) + shape.q_dim * shape.hidden + \
        3 * shape.hidden * shape.inter
    gemm = 2.0 * m * per_layer * shape.layers
    attn = 0.0
    for l in range(shape.layers):
        swa = (l % shape.swa_period) < shape.swa_period - 1
        for_span = sum(min(t + 1, shape.window) if (swa and shape.window) else t + 1 for t in range(m))
        attn += 2 * 2 * shape.n_q * shape.head_dim * for_span
    return gemm, attn


def prefill_report(shape, args, prefill_s: float) -> dict:
    """TTFT and MFMA utilisation of the prefill. mfma_util is the algorithmic
    FLOPs (GEMMs + causal attention) over TTFT over the dense bf16 peak.
    The GEMMs run two bf16 MFMA passes (activation hi and lo parts) and
    attention's QK^T and PV three (hi.hi, lo.hi, hi.lo): mfma_pass_frac is
    that matrix-core work, (2 gemm + 3 attn) / bf16 peak, over the TTFT."""
    gemm, attn = prefill_flops(shape, args.ctx)
    out = {"tokens": args.ctx, "ttft_ms": round(prefill_s * 1e3, 2),
           "algorithmic_tflop": round((gemm + attn) / 1e12, 3),
           "achieved_tflops": round((gemm + attn) / prefill_s / 1e12, 1)}
    if args.token_prefill:
        out["mode"] = "token by token (reference)"
        return out
    at_peak_s = (2 * gemm + 3 * attn) / (BF16_MFMA_PEAK_TFLOPS * 1e12)
    out.update({"mode": "batched: bf16 MFMA GEMMs (int8 weights exact in bf16, fp32 block scales, "
                        "activations as bf16 hi + lo) + flash attention on bf16 MFMA (hi + lo splits of "
                        "q, k, p and v; three products)",
                "gemm_tflop": round(gemm / 1e12, 3), "attention_tflop": round(attn / 1e12, 3),
                "mfma_util": round((gemm + attn) / prefill_s / (BF16_MFMA_PEAK_TFLOPS * 1e12), 4),
                "mfma_pass_time_at_peak_ms": round(at_peak_s * 1e3, 3),
                "mfma_pass_frac": round(at_peak_s / prefill_s, 4)})
    return out


class Hip:
    """The few HIP runtime calls the isolated-GEMV timing needs (ctypes; no torch)."""

    def __init__(self):
        import ctypes
        self.ct = ctypes
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def check(self, rc, what):
        if rc:
            raise RuntimeError(f"{what} failed: {rc}")

    def malloc(self, n):
        p = self.ct.c_void_p()
        self.check(self.h.hipMalloc(self.ct.byref(p), self.ct.c_size_t(n)), "hipMalloc")
        return p

    def h2d(self, dst, arr):
        a = np.ascontiguousarray(arr)
        self.check(self.h.hipMemcpy(dst, a.ctypes.data_as(self.ct.c_void_p), self.ct.c_size_t(a.nbytes), 1),
                   "hipMemcpy")

    def d2d(self, dst, src, n):
        self.check(self.h.hipMemcpy(dst, src, self.ct.c_size_t(n), 3), "hipMemcpy")

    def event(self):
        e = self.ct.c_void_p()
        self.check(self.h.hipEventCreate(self.ct.byref(e)), "hipEventCreate")
        return e

    def elapsed_ms(self, a, b):
        self.check(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = self.ct.c_float()
        self.check(self.h.hipEventElapsedTime(self.ct.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def free(self, p):
        self.h.hipFree(p)


def gemv_report(hip, launches: int = 200, rotate_bytes: int = 640 << 20):
    """The five isolated Q8_0 GEMV shapes of the 1B model through gg_q8_0_gemv
    (K -> N: fused QKV, O, gate+up, down, LM head), operands as the workload
    defines them (q uniform in [-127, 127], |d| lognormal, x ~ N(0, 1)). Each
    launch reads a different device copy of the weights, cycling over at
    least rotate_bytes (more than the 256 MB memory-side cache), so the bytes
    come from HBM; HIP events around `launches` back-to-back launches on one
    stream give the time per launch, launch gaps included. frac = algorithmic
    bytes (K N 34/32 + 4 K + 4 N) / time / 8 TB/s."""
    import ctypes
    L = capi.lib()
    out = {}
    for k, n in ((1152, 1536), (1024, 1152), (1152, 13824), (6912, 1152), (1152, 262144)):
        blocks, x = synth.gemv_operands(n, k, seed=n + k)
        psz = capi.lib().gg_q8_0_packed_size(n, k)
        copies = max(2, -(-rotate_bytes // psz))
        src = hip.malloc(blocks.nbytes)
        hip.h2d(src, blocks)
        w = hip.malloc(psz * copies)
        if L.gg_q8_0_repack(src, w, n, k, None):
            raise RuntimeError("gg_q8_0_repack failed")
        hip.check(hip.h.hipDeviceSynchronize(), "sync")
        for i in range(1, copies):
            hip.d2d(ctypes.c_void_p(w.value + i * psz), w, psz)
        dx, dy = hip.malloc(4 * k), hip.malloc(4 * n)
        hip.h2d(dx, x)
        e0, e1 = hip.event(), hip.event()
        for i in range(min(copies, 16)):   # warm-up
            L.gg_q8_0_gemv(ctypes.c_void_p(w.value + (i % copies) * psz), dx, dy, n, k, None)
        hip.check(hip.h.hipEventRecord(e0, None), "hipEventRecord")
        for i in range(launches):
            if L.gg_q8_0_gemv(ctypes.c_void_p(w.value + (i % copies) * psz), dx, dy, n, k, None):
                raise RuntimeError("gg_q8_0_gemv failed")
        hip.check(hip.h.hipEventRecord(e1, None), "hipEventRecord")
        us = hip.elapsed_ms(e0, e1) * 1e3 / launches
        nbytes = k * n // 32 * 34 + 4 * k + 4 * n
        out[f"{k}x{n}"] = {"us": round(us, 2), "bytes": nbytes, "GBs": round(nbytes / us / 1e3, 1),
                           "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                           "floor_us": round(nbytes / (HBM_PEAK_GBS * 1e9) * 1e6, 2), "weight_copies": copies}
        for p_ in (src, w, dx, dy):
            hip.free(p_)
    out["timing"] = (f"HIP events around {launches} back-to-back gg_q8_0_gemv launches on one stream, each on "
                     f"another device copy of the weights (>= {rotate_bytes >> 20} MiB cycled: HBM, not cache); "
                     "per-launch time includes the gap between launches")
    return out


def timed_decode(e, shape, tok, pos, steps, warmup, sample=(0.0, 0.9, 1.0), seed=0):
    """The generate() loop (one step queued ahead, each taking the previous id
    on the device) for `steps` timed steps after `warmup` synchronous ones;
    sampling options `sample` with seeded draws. Returns (tok/s, ms per step,
    mean algorithmic bytes per token, next position)."""
    rng = np.random.default_rng(seed)
    draw = (lambda: float(rng.random())) if sample[0] > 0 else (lambda: 0.0)
    for _ in range(warmup):
        tok = e.step(tok, pos, *sample, draw())
        pos += 1
    p0 = pos
    e.step_submit(tok, pos, *sample, draw())
    t0 = time.perf_counter()
    for _ in range(steps):
        e.step_submit(-1, pos + 1, *sample, draw())
        e.step_collect()
        pos += 1
    el = time.perf_counter() - t0
    e.step_collect()
    nbytes = float(np.mean([step_bytes(shape, q) for q in range(p0, p0 + steps)]))
    return steps / el, el * 1e3 / steps, nbytes, pos + 1


def decode_entry(tok_s, ms, nbytes, extra=None):
    d = {"tok_s": round(tok_s, 2), "ms_per_step": round(ms, 4), "bytes_per_token": int(nbytes),
         "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    d.update(extra or {})
    return d


def extra_workloads(shape, tensors, args) -> dict:
    """The other configurations the reference's benchmark and the workload
    set name, each driver-timed in this run with its own HBM fraction:
    sampled decode at 2K (generate()'s defaults T 0.7, top-p 0.9, repetition
    1.2), reference attention mode at 2K (the JavaScript host's default), the
    270M model (64-id prompt, 128 greedy steps), the five isolated GEMVs, and
    sampled decode at 32K KV after three chained turns with KV reuse."""
    out = {}
    steps = min(args.steps, 128)
    prompt = synth.prompt_ids(2048, seed=2048, vocab=shape.vocab)
    sample = (0.7, 0.9, 1.2)

    # 1B at 2K: sampled (the same weights and attention as the headline run)
    e = capi.Engine(shape.gg_config(prefill_batch=2048))
    e.upload_model(tensors)
    e.finalize()
    e.penalty_reset()
    e.penalty_add(prompt)
    e.prefill(prompt, 0)
    tok = e.select(*sample, 0.5)
    r = timed_decode(e, shape, tok, 2048, steps, 8, sample, seed=7)
    out["decode_1b_2k_sampled"] = decode_entry(*r[:3], {"sampling": "T 0.7, top-p 0.9, repetition 1.2, seeded u",
                                                         "decode_path": e.decode_path()})
    e.close()
    print(f"# sampled 2K: {r[0]:.1f} tok/s", file=sys.stderr, flush=True)

    # 1B at 2K, reference attention mode (full attention, theta 1e6 on every layer)
    rs = shape.reference_mode()
    e = capi.Engine(rs.gg_config(prefill_batch=2048))
    e.upload_model(tensors)
    e.finalize()
    e.prefill(prompt, 0)
    tok = e.select()
    r = timed_decode(e, rs, tok, 2048, steps, 8)
    out["decode_1b_2k_reference_mode"] = decode_entry(*r[:3], {"attention": "full on all 26 layers, theta 1e6",
                                                               "decode_path": e.decode_path()})
    e.close()
    print(f"# reference mode 2K: {r[0]:.1f} tok/s", file=sys.stderr, flush=True)

    # 270M: 64-id prompt, TTFT, then 128 greedy steps (contextLength 2048)
    s270 = synth.GEMMA3_270M.with_ctx(2048).gemma3_mode()
    t270 = synth.make_model(s270, seed=270)
    p64 = synth.prompt_ids(64, seed=64, vocab=s270.vocab)
    e = capi.Engine(s270.gg_config(prefill_batch=64))
    e.upload_model(t270)
    e.finalize()
    ttft = []
    for _ in range(3):
        e.reset_kv()
        t0 = time.perf_counter()
        e.prefill(p64, 0)
        tok = e.select()
        ttft.append(time.perf_counter() - t0)
    r = timed_decode(e, s270, tok, 64, 128, 0)
    out["decode_270m"] = decode_entry(*r[:3], {"prompt": 64, "steps": 128, "ttft_ms": round(min(ttft) * 1e3, 3),
                                               "decode_path": e.decode_path()})
    e.close()
    del t270
    print(f"# 270M: {r[0]:.1f} tok/s, TTFT {min(ttft) * 1e3:.2f} ms", file=sys.stderr, flush=True)

    # isolated GEMVs
    out["gemv_1b_shapes"] = gemv_report(Hip())
    print("# GEMV shapes done", file=sys.stderr, flush=True)

    # 32K: three chained turns (16384 + 8192 + 8100 prompt ids, 7 sampled steps
    # each as generate() writes them), then sampled decode at ~32.7K positions
    s32 = shape.with_ctx(32768)
    e = capi.Engine(s32.gg_config(prefill_batch=4096))
    e.upload_model(tensors)
    e.finalize()
    rng = np.random.default_rng(55)
    kv_pos, tok = 0, 0
    t0 = time.perf_counter()
    for turn, n in enumerate((16384, 8192, 8100)):
        p = synth.prompt_ids(n, seed=300 + turn, vocab=s32.vocab)
        e.penalty_reset()
        e.penalty_add(p)
        e.prefill(p, kv_pos)
        kv_pos += n
        tok = e.select(*sample, float(rng.random()))
        for _ in range(7):
            tok = e.step(tok, kv_pos, *sample, float(rng.random()))
            kv_pos += 1
    fill_s = time.perf_counter() - t0
    n32 = min(steps, 64)
    r = timed_decode(e, s32, tok, kv_pos, n32, 0, sample, seed=56)
    out["decode_1b_32k_sampled"] = decode_entry(*r[:3], {"positions": [kv_pos, kv_pos + n32 - 1],
                                                         "turns": "16384 + 8192 + 8100 prompt ids, 7 sampled "
                                                                  "steps each, KV reused across turns",
                                                         "three_turn_fill_s": round(fill_s, 3),
                                                         "decode_path": e.decode_path()})
    e.close()
    print(f"# 32K sampled: {r[0]:.1f} tok/s", file=sys.stderr, flush=True)
    return out


def copy_calibration(nbytes: int):
    """One device-to-device copy of nbytes (the runtime's copy kernel): the
    reference point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to
    HBM bytes."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), ctypes.c_size_t(nbytes)) or hip.hipMalloc(ctypes.byref(b), ctypes.c_size_t(nbytes)):
        raise RuntimeError("hipMalloc failed")
    hip.hipMemset(a, 1, ctypes.c_size_t(nbytes))
    hip.hipMemcpy(b, a, ctypes.c_size_t(nbytes), 3)   # hipMemcpyDeviceToDevice
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)


def measured_traffic(name: str):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, scaled by the copy
    calibration)."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch"):
                return int(line.split()[1])
    except OSError:
        pass
    return None


def _oracle_rate(o, pos0: int, budget_s: float, select: bool):
    """Steps per second of the oracle over at least two steps and budget_s."""
    n, t0, tok = 0, time.perf_counter(), 2
    while True:
        o.forward(tok, pos0 + n)
        if select:
            tok = o.select(0.0, 0.9, 1.0, 0.0)
        n += 1
        el = time.perf_counter() - t0
        if n >= 2 and el >= budget_s:
            return n, el


def cpu_baseline(shape, tensors, pos0: int, budget_s: float, threads: int):
    """The C oracle (a restatement of the reference pipeline in fp32) on the
    host: greedy decode on `threads` cores (the reported value), the same on
    one core, and forward passes without the LM head (the reference's
    token-by-token prefill) whose rate gives an extrapolated 2048-token TTFT."""
    from oracle import oracle as orc
    orc.set_threads(threads)
    o = orc.OracleModel(shape, tensors)
    n, el = _oracle_rate(o, pos0, budget_s, True)
    cores = orc.get_threads()
    nf, elf = _oracle_rate(o, pos0 + n, max(2.0, budget_s / 5), False)
    orc.set_threads(1)
    n1, el1 = _oracle_rate(o, pos0 + n + nf, max(2.0, budget_s / 5), True)
    orc.set_threads(threads)
    o.close()
    return {"value": n / el, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode steps (forward + LM head + argmax) of the 1B shape at positions "
                      f"{pos0}..{pos0 + n - 1} over a zero-filled KV cache, C oracle with OpenMP over "
                      f"output rows, {el:.1f} s",
            "value_1core": round(n1 / el1, 3),
            "sample_1core": f"{n1} greedy decode steps on one core, {el1:.1f} s",
            "prefill_tok_s": round(nf / elf, 3),
            "ttft_2048_extrapolated_s": round(2048 * elf / nf, 1),
            "sample_prefill": f"{nf} forward passes without the LM head on {cores} cores, {elf:.1f} s; "
                              f"TTFT of a 2048-token prompt extrapolated from their rate"}


def prefill_rows(args) -> int:
    """Rows per batched prefill slice (0 = token by token)."""
    if args.token_prefill:
        return 0
    return args.prefill_batch or min(args.ctx, 4096)


def probe_kernel(shape, tensors, prompt, args):
    """Mean device time (ms) of the probed kernel and of an empty event pair
    over args.probe_steps decode steps whose kernels are launched directly."""
    had = os.environ.get("GG_NO_GRAPH")
    os.environ["GG_NO_GRAPH"] = "1"
    try:
        e = capi.Engine(shape.gg_config(prefill_batch=prefill_rows(args)))
        e.set_decode_path("graph")
        e.set_probe(args.probe, args.probe_layer)
        e.upload_model(tensors)
        e.finalize()
    finally:
        if had is None:
            del os.environ["GG_NO_GRAPH"]
    e.prefill(prompt, 0)
    e.set_timing(True)   # same event traffic per step as the device-time loop
    tok = e.select()
    pos = args.ctx
    for _ in range(4):
        tok = e.step(tok, pos)
        pos += 1
    br, em = [], []
    for _ in range(args.probe_steps):
        tok = e.step(tok, pos)
        br.append(e.probe_elapsed_ms())
        em.append(e.probe_overhead_ms())
        pos += 1
    e.close()
    return float(np.mean(br)), float(np.mean(em))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=2048, help="context positions filled before decoding")
    ap.add_argument("--probe", default="gate_up", choices=["none", "qkv", "o", "gate_up", "down", "lm_head"])
    ap.add_argument("--probe-layer", type=int, default=13,
                    help="layer of the probed kernel: deep enough into the step that the host has queued it before the GPU gets there")
    ap.add_argument("--probe-steps", type=int, default=64, help="timed steps of the kernel-timing loop")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--reference-mode", action="store_true", help="full attention, one theta (src/ as shipped)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="run one device-to-device copy of BYTES first (PMC calibration runs)")
    ap.add_argument("--prefill-batch", type=int, default=0,
                    help="rows per batched prefill slice (default: the whole context, at most 4096)")
    ap.add_argument("--token-prefill", action="store_true",
                    help="fill the context token by token (the reference's prefillBatched) instead of batched")
    ap.add_argument("--decode", default="fused", choices=["fused", "graph"],
                    help="decode path: the persistent kernel (one launch per token) or one kernel per phase")
    ap.add_argument("--sync-steps", action="store_true",
                    help="time synchronous gg_step calls instead of the pipelined loop the JS host runs")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the other workloads (sampled, reference mode, 270M, GEMV shapes, 32K)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the batch-1 token loop runs on "
              f"a single MI355X, and more GPUs serve more independent conversations (one context per GPU, no "
              f"exchange) rather than one faster one", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
    # positions decoded past the context: the timed engine's warm-up, timed and
    # device-timing steps, or the kernel-timing engine's 4 + probe_steps
    # positions used after the prompt: warm-up, the timed steps and the one
    # queued past them, the synchronous reference loop, the event-timed loop
    after = args.warmup + args.steps + 1 + min(args.steps, 128) + min(args.steps, 64)
    ctx_len = max(4096, args.ctx + max(after, 4 + args.probe_steps) + 8)
    shape = synth.GEMMA3_1B.with_ctx(ctx_len)
    shape = shape.reference_mode() if args.reference_mode else shape.gemma3_mode()
    t0 = time.perf_counter()
    tensors = synth.make_model(shape, seed=1)
    t_gen = time.perf_counter() - t0
    cfg = shape.gg_config(prefill_batch=prefill_rows(args))
    e = capi.Engine(cfg)
    e.set_decode_path(args.decode)
    e.upload_model(tensors)
    e.finalize()
    decode_path = e.decode_path()
    print(f"# model ready: generate {t_gen:.1f}s, upload {time.perf_counter() - t0 - t_gen:.1f}s", file=sys.stderr,
          flush=True)

    prompt = synth.prompt_ids(args.ctx, seed=2048, vocab=shape.vocab)
    ttft = []
    for rep in range(1 if args.token_prefill else 5):   # TTFT: prefill + first token, best of 5
        e.reset_kv()
        t0 = time.perf_counter()
        e.prefill(prompt, 0)
        tok = e.select()
        ttft.append(time.perf_counter() - t0)
    prefill_s = min(ttft)
    print(f"# prefill {args.ctx} tokens + first select: {prefill_s * 1e3:.1f} ms", file=sys.stderr, flush=True)

    pos = args.ctx
    for _ in range(args.warmup):
        tok = e.step(tok, pos)
        pos += 1
    pos_timed0 = pos
    if args.sync_steps:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            tok = e.step(tok, pos)
            pos += 1
        elapsed = time.perf_counter() - t0
    else:
        # the JavaScript host's generate() loop: one step queued ahead, each
        # step taking the previous step's id on the device (gg_step_submit
        # with token -1); every timed step is collected by the host
        e.step_submit(tok, pos)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            e.step_submit(-1, pos + 1)
            tok = e.step_collect()
            pos += 1
        elapsed = time.perf_counter() - t0
        e.step_collect()   # the step queued past the timed ones
        pos += 1
    pos_timed1 = pos_timed0 + args.steps
    # synchronous gg_step calls (one host round trip per step), for reference
    n_sync = min(args.steps, 128)
    t0 = time.perf_counter()
    for _ in range(n_sync):
        tok = e.step(tok, pos)
        pos += 1
    sync_ms = (time.perf_counter() - t0) * 1e3 / n_sync
    # device time per step from the engine's step events, in a separate
    # untimed loop (the three event records cost ~9 us of device time a step)
    e.set_timing(True)
    fwd_ms = []
    for _ in range(min(args.steps, 64)):
        tok = e.step(tok, pos)
        fwd_ms.append(sum(e.last_timing()))
        pos += 1
    e.close()

    value = args.steps / elapsed
    ms_per_step = elapsed * 1e3 / args.steps
    avg_bytes = float(np.mean([step_bytes(shape, p) for p in range(pos_timed0, pos_timed1)]))
    dev_ms = float(np.mean(fwd_ms))

    # the committed counter summaries were taken on the default workload
    # (gemma3 attention, 2048 positions); other workloads report no traffic
    default_workload = args.ctx == 2048 and not args.reference_mode
    if decode_path == "fused":
        # the persistent kernel is the whole token: one launch per gg_step,
        # timed by the engine's step events (forward = the launch)
        k_ms = dev_ms
        k_bytes = int(avg_bytes)
        variant = "true" if ctx_len > 4096 else "false"   # the long-span variant above 4096 positions
        roof = {"bound": "hbm",
                "kernel": f"k_decode<DEC_STEP, {variant}, false> (persistent, greedy copy: 26 layers + LM head + "
                          "selection)",
                "achieved": round(k_bytes / (k_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(k_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic("decode_step_traffic.txt") if default_workload else None,
                "bytes_per_launch": k_bytes,
                "avg_launch_us": round(k_ms * 1e3, 2), "launches": len(fwd_ms),
                "timing": "HIP events around each k_decode launch (the step's inputs are kernel arguments) over "
                          f"{len(fwd_ms)} decode steps"}
    else:
        # dominant-kernel timing: the same forward pass with its kernels
        # launched directly on the engine's stream (the form rocprofv3 traces),
        # HIP events recorded around the probed launch in every step of a timed
        # loop, and an empty event pair recorded right before it
        probe = args.probe if args.probe != "none" else "gate_up"
        k_bytes = kernel_bytes(shape, probe, pos_timed0)
        bracket_ms = empty_ms = float("nan")
        if args.probe != "none":
            bracket_ms, empty_ms = probe_kernel(shape, tensors, prompt, args)
        k_ms = bracket_ms
        achieved = k_bytes / (k_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": f"{args.probe} GEMV (layer {args.probe_layer})",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gate_up_gemv_traffic.txt") if default_workload else None,
                "bytes_per_launch": k_bytes, "avg_launch_us": round(k_ms * 1e3, 2),
                "empty_event_pair_us": round(empty_ms * 1e3, 2), "launches": args.probe_steps,
                "timing": "HIP events around each direct launch of the kernel over a timed loop of "
                          f"{args.probe_steps} decode steps"}
    out = {
        "metric": METRIC if args.ctx == 2048 else METRIC.replace("@ctx2k", f"@ctx{args.ctx}"),
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32; decode FFN activations as 3 int8 planes per 32-block (within 2e-7 of the block max), "
                 "int32-exact products",
        "data": "synthetic: seeded random-init Q8_0 weights of the Gemma-3-1B architecture, seeded uniform ids",
        "config": {"workload": f"gemma3-1b-q8_0-greedy-decode-after-{args.ctx}", "ctx_prefilled": args.ctx,
                   "batch": 1, "attention": "reference (full, theta 1e6)" if args.reference_mode else
                   "gemma3 (22 local layers window 512 theta 1e4, 4 global theta 1e6)",
                   "positions": [pos_timed0, pos_timed1 - 1], "decode_path": decode_path,
                   "step_loop": "gg_step per step" if args.sync_steps else
                   "gg_step_submit one step ahead (input id taken on the device) + gg_step_collect, as the "
                   "JavaScript host's generate() runs"},
        "ms_per_step_sync": round(sync_ms, 4),
        "roofline": roof,
        "step_roofline": {"bytes_per_token": int(avg_bytes),
                          "achieved_GBs": round(avg_bytes / (ms_per_step * 1e-3) / 1e9, 1),
                          "frac": round(avg_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          "device_ms_per_step": round(dev_ms, 4)},
        "prefill": prefill_report(shape, args, prefill_s),
    }
    if not args.no_extras and args.ctx == 2048 and not args.reference_mode and decode_path == "fused":
        out["workloads"] = extra_workloads(shape, tensors, args)
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        try:
            out["cpu_baseline"] = cpu_baseline(shape, tensors, args.ctx, args.cpu_seconds, threads)
        except Exception as ex:  # the oracle is optional for the GPU number
            out["cpu_baseline"] = {"error": str(ex)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
