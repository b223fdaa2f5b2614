#!/usr/bin/env python3
"""Fine-tuning step throughput on one MI355X: Qwen2.5-1.5B-architecture decoder (fp32 weights, gradients and AdamW
state; random-init seeded Gaussians), one full step = forward + backward over batch 8 x seq 1024 random tokens with
next-token cross-entropy, global-norm clipping and AdamW, bit-identical to the reference CPU kernels.

Prints one JSON line (the driver's contract): tokens/s of whole steps with inputs already resident in HBM, the
roofline of the dominant kernel (the FP64-FMA matmul, timed live with a pair of HIP events on its stream around
every launch, over as many steps again run right after the timed ones: the events cost the small configs several
percent of their step, so the throughput steps run without them) and the reference CPU path timed on this host's
cores for a bounded sample of the same step.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3|c1] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP64_PEAK_TFLOPS = 78.6  # MI355X dense FP64 (vector FMA and matrix alike)

CONFIGS = {
    # the metric's workload
    "c3": dict(name="Qwen2.5-1.5B", vocab=151936, hidden=1536, intermediate=8960, layers=28, heads=12, kv_heads=2,
               head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, tie_embeddings=True, attention_bias=True,
               batch=8, seq=1024),
    # the reference's CPU-runnable case
    "c1": dict(name="SmolLM2-135M", vocab=49152, hidden=576, intermediate=1536, layers=30, heads=9, kv_heads=3,
               head_dim=64, rms_norm_eps=1e-5, rope_theta=1e5, tie_embeddings=True, attention_bias=False,
               batch=4, seq=256),
    # LoRA (rank 16, alpha 32, q k v o gate up down; A ~ N(0, 0.02), B = 0) on a Q8_0 base
    "c4": dict(name="Qwen3-0.6B LoRA on a Q8_0 base", vocab=151936, hidden=1024, intermediate=3072, layers=28,
               heads=16, kv_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6, tie_embeddings=True,
               attention_bias=False, qk_norm=1, batch=8, seq=2048,
               lora=dict(rank=16, alpha=32.0, targets=("q", "k", "v", "o", "gate", "up", "down"))),
    # routed experts with the load-balancing loss (router_aux_loss 0.01)
    "c5": dict(name="OLMoE-1B-7B", vocab=50304, hidden=2048, intermediate=1024, layers=16, heads=16, kv_heads=16,
               head_dim=128, rms_norm_eps=1e-5, rope_theta=1e4, tie_embeddings=False, attention_bias=False,
               qk_norm=2, experts=64, experts_per_token=8, normalize_expert_weights=False, expert_intermediate=1024,
               router_aux_loss=0.01, batch=4, seq=2048),
}

METRIC = "finetune tokens/s, Qwen2.5-1.5B fp32 step, bit-exact vs CPU; % of roofline"
SEED = 0
LEARNING_RATE = 1e-4  # schedule "constant", betas 0.9 / 0.999, eps 1e-8, weight decay 0.01, max_grad_norm 1.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def natural_key(name: str):
    import re

    parts = re.split(r"(\d+)", name)
    return (*((0, int(p), "") if p.isdigit() else (1, 0, p) for p in parts), name)


def init_weights(trainer, lib, shapes: dict[str, tuple[int, ...]]) -> None:
    """fill_gaussian(SEED * 1000 + i) * 0.02f per tensor, i its index in natural name order; norm weights 1.0."""
    names = sorted(shapes, key=natural_key)

    def one(item):
        index, name = item
        n = int(np.prod(shapes[name]))
        if name.endswith("norm.weight"):
            values = np.ones(n, np.float32)
        else:
            values = np.empty(n, np.float32)
            rc = lib.dllm_hip_fill_gaussian(C.c_uint64(SEED * 1000 + index), values.ctypes.data_as(C.c_void_p),
                                            C.c_size_t(n), C.c_float(0.02))
            assert rc == 0
        trainer.set(name, values)

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
        list(pool.map(one, enumerate(names)))


def tensor_shapes(cfg) -> dict[str, tuple[int, ...]]:
    H, q, kv, inter = cfg["hidden"], cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"], cfg["intermediate"]
    shapes = {"token_embedding.weight": (cfg["vocab"], H), "final_norm.weight": (H,)}
    experts, ei = cfg.get("experts", 0), cfg.get("expert_intermediate", 0) or inter
    for i in range(cfg["layers"]):
        p = f"layers.{i}."
        shapes.update({p + "attention_norm.weight": (H,), p + "attention.q.weight": (q, H),
                       p + "attention.k.weight": (kv, H), p + "attention.v.weight": (kv, H),
                       p + "attention.o.weight": (H, q), p + "mlp_norm.weight": (H,)})
        if experts:
            shapes[p + "mlp.router.weight"] = (experts, H)
            for e in range(experts):
                x = f"{p}mlp.experts.{e}."
                shapes.update({x + "gate.weight": (ei, H), x + "up.weight": (ei, H), x + "down.weight": (H, ei)})
        else:
            shapes.update({p + "mlp.gate.weight": (inter, H), p + "mlp.up.weight": (inter, H),
                           p + "mlp.down.weight": (H, inter)})
        if cfg.get("qk_norm"):
            per_head = cfg["qk_norm"] == 1
            shapes.update({p + "attention.q_norm.weight": (cfg["head_dim"] if per_head else q,),
                           p + "attention.k_norm.weight": (cfg["head_dim"] if per_head else kv,)})
        if cfg["attention_bias"]:
            shapes.update({p + "attention.q.bias": (q,), p + "attention.k.bias": (kv,), p + "attention.v.bias": (kv,)})
    if not cfg["tie_embeddings"]:
        shapes["lm_head.weight"] = (cfg["vocab"], H)
    return shapes


def init_adapters(trainer, lib, cfg) -> None:
    """LoRA adapters: A = fill_gaussian(SEED * 1000 + 500000 + i) * 0.02f (i its index among the adapters in
    natural order), B = 0."""
    names = sorted((n for n in trainer.names if n.endswith((".lora_a", ".lora_b"))), key=natural_key)
    for i, name in enumerate(names):
        ptr, numel = trainer._tensor(name, trainer.PARAM)
        values = np.zeros(numel, np.float32)
        if name.endswith(".lora_a"):
            assert lib.dllm_hip_fill_gaussian(C.c_uint64(SEED * 1000 + 500000 + i), values.ctypes.data_as(C.c_void_p),
                                              C.c_size_t(numel), C.c_float(0.02)) == 0
        trainer.set(name, values)


def make_windows(lib, cfg, step: int) -> list[list[int]]:
    """Random(SEED + step).next_u64() % vocab, batch windows of seq + 1 tokens."""
    n = cfg["batch"] * (cfg["seq"] + 1)
    tokens = np.empty(n, np.int64)
    assert lib.dllm_hip_random_tokens(C.c_uint64(SEED + step), tokens.ctypes.data_as(C.c_void_p), C.c_size_t(n),
                                      C.c_int64(cfg["vocab"])) == 0
    w = cfg["seq"] + 1
    return [tokens[i * w:(i + 1) * w].tolist() for i in range(cfg["batch"])]


def matmul_flops_per_step(cfg) -> float:
    """Algorithmic matmul work of one step: 6 x matmul parameters a token passes through x tokens (forward, dX, dW);
    a routed layer counts its router and experts_per_token experts."""
    H, q, kv, inter, V = (cfg["hidden"], cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"],
                          cfg["intermediate"], cfg["vocab"])
    if cfg.get("experts"):
        mlp = cfg["experts"] * H + cfg["experts_per_token"] * 3 * H * (cfg.get("expert_intermediate") or inter)
    else:
        mlp = 3 * H * inter
    per_layer = H * q * 2 + H * kv * 2 + mlp
    params = cfg["layers"] * per_layer + V * H
    return 6.0 * params * cfg["batch"] * cfg["seq"]


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_sample(O, kern, cfg, T: int, head_rows: int, n_opt: int):
    """Seconds of (one window of T tokens through a 1-layer model of this architecture, vocab 4096), (the head at
    head_rows vocabulary rows over T rows: linear, cross-entropy, linear_backward) and (sum_squares + adamw_step on
    n_opt elements)."""
    H = cfg["hidden"]
    small = O.Decoder("sample", vocab=4096, hidden=H, inter=cfg["intermediate"], layers=1, heads=cfg["heads"],
                      kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"], eps=cfg["rms_norm_eps"],
                      rope_theta=cfg["rope_theta"], tied=cfg["tie_embeddings"], attn_bias=cfg["attention_bias"],
                      qk_norm=cfg.get("qk_norm", 0), experts=cfg.get("experts", 0),
                      topk=cfg.get("experts_per_token", 0), normalize=cfg.get("normalize_expert_weights", False),
                      expert_inter=cfg.get("expert_intermediate", 0))
    weights = O.synthetic_weights(small, seed=SEED, scale=0.02)
    rng = O.Random(SEED)
    tokens = [rng.next_u64() % small.vocab for _ in range(T + 1)]
    t0 = time.perf_counter()
    O.window_gradients(kern, small, weights, tokens[:-1], tokens[1:], scale=1.0 / T,
                       router_scale=cfg.get("router_aux_loss", 0.0) / cfg["batch"])
    t_window = time.perf_counter() - t0
    hidden = O.gaussian(SEED + 1, T, H)
    head = O.gaussian(SEED + 2, head_rows, H, scale=0.02)
    targets = np.array([rng.next_u64() % head_rows for _ in range(T)], np.int64)
    t0 = time.perf_counter()
    logits = kern.linear(hidden, head)
    _, dlogits = kern.cross_entropy(logits, targets, 1.0 / T)
    kern.linear_backward(hidden, head, dlogits)
    t_head = time.perf_counter() - t0
    p, g = O.gaussian(SEED + 3, n_opt, scale=0.02), O.gaussian(SEED + 4, n_opt, scale=1e-3)
    m, v = np.zeros(n_opt, np.float32), np.zeros(n_opt, np.float32)
    t0 = time.perf_counter()
    kern.sum_squares(g)
    kern.adamw_step(p, g, m, v, 1e-4, 0.9, 0.999, 1e-8, 0.01, 0.1, 0.001, 1.0)
    t_opt = time.perf_counter() - t0
    return t_window, t_head, t_opt


def cpu_baseline(cfg) -> dict | None:
    """The reference CPU path (its own kernels from oracle/_ref, or the oracle's C restatement when that library is
    absent), driven by the oracle's step orchestration, timed on a bounded sample of the step and scaled to it, with
    the reference's thread pool at this host's cores (nproc, capped at the 16 cores a one-GPU box grants a job) and
    again at 1 thread:
      one window of T tokens through a 1-layer model of this architecture with a 4096-token vocabulary;
      the head (linear, cross-entropy, linear_backward) at R vocabulary rows over T rows, scaled to the vocab;
      adamw_step and sum_squares on N elements, scaled to the parameter count.
    step = batch x (seq / T) x (layers x (window - head share) + head x vocab / R) + optimizer x params / N.
    The many-thread sample is T = 1024, R = 8192, N = 16M; the 1-thread one T = 256, R = 2048, N = 4M."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O

    kind = "reference" if O.reference_available() else "port"
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = min(16, nproc) if kind == "reference" else 1
    kern = O.ref_kernels() if kind == "reference" else O.oracle_kernels()
    params = sum(int(np.prod(s)) for s in tensor_shapes(cfg).values())
    if "lora" in cfg:  # AdamW runs over the adapters only
        H, q, kv, inter = cfg["hidden"], cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"], cfg["intermediate"]
        params = cfg["layers"] * cfg["lora"]["rank"] * (2 * (H + q) + 2 * (H + kv) + 3 * (H + inter))
    V, tokens_per_step = cfg["vocab"], cfg["batch"] * cfg["seq"]

    def extrapolate(T, R, N, t_window, t_head, t_opt):
        stretch = cfg["seq"] / T  # a window longer than the sample: linear in tokens (understates the attention)
        layer = t_window - t_head * 4096 / R
        return cfg["batch"] * stretch * (cfg["layers"] * layer + t_head * V / R) + t_opt * params / N

    runs = {}
    for n_threads, (T, R, N) in ((threads, (min(cfg["seq"], 1024), 8192, 16 << 20)), (1, (256, 2048, 4 << 20))):
        if kind == "reference":
            O.ref().ref_set_threads(C.c_size_t(n_threads))
        times = _cpu_sample(O, kern, cfg, T, R, N)
        runs[n_threads] = (T, R, N, times, extrapolate(T, R, N, *times))
    T, R, N, (t_window, t_head, t_opt), step = runs[threads]
    step1 = runs[1][4]
    return {
        "value": tokens_per_step / step,
        "unit": "tokens/s",
        "cores": threads,
        "kind": kind,
        "value_1_thread": tokens_per_step / step1,
        "nproc": nproc,
        "cpu_model": _cpu_model(),
        "sample": (f"{threads} threads of {nproc} ({_cpu_model()}): 1-layer {cfg['name']}-shaped model, 1 window x {T} "
                   f"tokens, vocab 4096 ({t_window:.2f} s); head at {R} vocab rows ({t_head:.2f} s); optimizer on "
                   f"{N} params ({t_opt:.2f} s); scaled to {cfg['layers']} layers, {cfg['seq']}-token windows, vocab "
                   f"{V}, batch {cfg['batch']}, {params} params: {step:.1f} s per step (extrapolated)"
                   + ("; the base's gradients stand for the LoRA step" if "lora" in cfg else "")
                   + f". 1 thread (T {runs[1][0]}, {runs[1][1]} head rows, {runs[1][2]} params): {step1:.1f} s per step"),
    }


COPY_BYTES = 1 << 30


def copy_calibration() -> int:
    """A plain copy kernel of known size (the library's dllm_hip_copy of 1 GiB), three times: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE give the counters' scale against bytes actually moved."""
    from etalii_dllm_amd import kernels as K

    src, dst = K.Device(COPY_BYTES), K.Device(COPY_BYTES)
    K.check(K.lib.dllm_hip_memset(src.ptr, 1, COPY_BYTES))
    for _ in range(3):
        K.check(K.lib.dllm_hip_copy(dst.ptr, src.ptr, COPY_BYTES, None))
    K.check(K.lib.dllm_hip_synchronize())
    return 0


def _counter_rows(path: str, kernel_substring: str, counter: str) -> list[float]:
    import csv

    out = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if kernel_substring in row["Kernel_Name"] and row["Counter_Name"] == counter:
                out.append(float(row["Counter_Value"]))
    return out


def traffic_summary(config: str, fetch_csv: str, write_csv: str, copy_fetch_csv: str, copy_write_csv: str) -> int:
    """HBM bytes per matmul launch = mean(FETCH_SIZE) x fetch scale + mean(WRITE_SIZE) x write scale, the scales
    being the copy kernel's known bytes over what the same counters read for it (counters are in KiB)."""
    fetch = _counter_rows(fetch_csv, "gemm_mfma_kernel", "FETCH_SIZE")
    write = _counter_rows(write_csv, "gemm_mfma_kernel", "WRITE_SIZE")
    copy_fetch = max(_counter_rows(copy_fetch_csv, "copy", "FETCH_SIZE") or
                     _counter_rows(copy_fetch_csv, "elementwise", "FETCH_SIZE"))
    copy_write = max(_counter_rows(copy_write_csv, "copy", "WRITE_SIZE") or
                     _counter_rows(copy_write_csv, "elementwise", "WRITE_SIZE"))
    fetch_scale = COPY_BYTES / (copy_fetch * 1024.0)
    write_scale = COPY_BYTES / (copy_write * 1024.0)
    per_launch = (sum(fetch) / len(fetch) * 1024.0 * fetch_scale + sum(write) / len(write) * 1024.0 * write_scale)
    path = ROOT / "profiles" / "gemm_traffic.json"
    data = json.loads(path.read_text()) if path.exists() else {}
    data[config] = {"bytes_per_launch": per_launch, "launches": len(fetch), "fetch_scale": fetch_scale,
                    "write_scale": write_scale, "fetch_kib_mean": sum(fetch) / len(fetch),
                    "write_kib_mean": sum(write) / len(write)}
    path.write_text(json.dumps(data, indent=1) + "\n")
    print(json.dumps(data[config]))
    return 0


def kernel_suite(iters: int = 20) -> int:
    """The per-kernel entry points beyond the step (quantised inference linears, encoder/T5 kernels), each on
    device-resident inputs: time per call over `iters` back-to-back calls after 3 warmups, and the rate against the
    bound that applies. One JSON line per case on stdout."""
    from etalii_dllm_amd import kernels as K

    lib, rng = K.lib, np.random.default_rng(0)

    def timed(run) -> float:
        for _ in range(3):
            run()
        K.check(lib.dllm_hip_synchronize())
        t = time.perf_counter()
        for _ in range(iters):
            run()
        K.check(lib.dllm_hip_synchronize())
        return (time.perf_counter() - t) / iters

    def report(case: str, seconds: float, **rates) -> None:
        print(json.dumps({"kernel_suite": case, "us_per_call": round(seconds * 1e6, 2), **rates}), flush=True)

    hbm, fp64_lane_ops = 8.0e12, 78.6e12 / 2  # bytes/s; vector FP64 instructions x 64 lanes per second
    for rows, inf, outf in [(1, 1536, 8960), (1, 8960, 1536), (8, 4096, 4096), (512, 1536, 8960), (4096, 1536, 8960)]:
        x = K.Device.of(rng.standard_normal((rows, inf)).astype(np.float32))
        q, sc = K.quantize_q8_0((rng.standard_normal((outf, inf)) * 0.02).astype(np.float32))
        dq, ds, out = K.Device.of(q), K.Device.of(sc), K.Device(rows * outf * 4)
        ws = K.Device(lib.dllm_hip_linear_q8_workspace(rows, inf))
        t = timed(lambda: K.check(lib.dllm_hip_linear_q8(x.ptr, dq.ptr, ds.ptr, None, out.ptr, rows, inf, outf, ws.ptr,
                                                         ws.nbytes, None)))
        weight_bytes = q.nbytes + sc.nbytes
        combine = 4.0 * rows * outf * (inf // 32) / fp64_lane_ops  # scale product, conversion, multiply, add
        report(f"linear_q8 rows={rows} in={inf} out={outf}", t, weights_GBps=round(weight_bytes / t / 1e9, 1),
               hbm_frac=round(weight_bytes / t / hbm, 3), int8_equiv_TOPs=round(2 * rows * inf * outf / t / 1e12, 2),
               combine_bound_frac=round(combine / t, 3))
    for rows, inf, outf in [(1, 1536, 8960), (1, 8960, 1536)]:
        x = K.Device.of(rng.standard_normal((rows, inf)).astype(np.float32))
        pk, sc = K.quantize_q4_0((rng.standard_normal((outf, inf)) * 0.02).astype(np.float32))
        dq, ds, out = K.Device.of(pk), K.Device.of(sc), K.Device(rows * outf * 4)
        ws = K.Device(lib.dllm_hip_linear_q4_workspace(rows, inf, outf))
        t = timed(lambda: K.check(lib.dllm_hip_linear_q4(x.ptr, dq.ptr, ds.ptr, None, out.ptr, rows, inf, outf, ws.ptr,
                                                         ws.nbytes, None)))
        weight_bytes = pk.nbytes + sc.nbytes
        report(f"linear_q4 rows={rows} in={inf} out={outf}", t, weights_GBps=round(weight_bytes / t / 1e9, 1),
               hbm_frac=round(weight_bytes / t / hbm, 3))
    n = 1 << 24
    x = K.Device.of(rng.standard_normal(n).astype(np.float32))
    o = K.Device(n * 4)
    t = timed(lambda: K.check(lib.dllm_hip_gelu(x.ptr, o.ptr, n, None)))
    report(f"gelu n={n}", t, GBps=round(8 * n / t / 1e9, 1), Gelem_per_s=round(n / t / 1e9, 2))
    t = timed(lambda: K.check(lib.dllm_hip_gelu_backward(x.ptr, x.ptr, o.ptr, n, None)))
    report(f"gelu_backward n={n}", t, GBps=round(12 * n / t / 1e9, 1), Gelem_per_s=round(n / t / 1e9, 2))
    for rows, dim in [(4096, 768), (16384, 1024)]:
        x = K.Device.of(rng.standard_normal((rows, dim)).astype(np.float32))
        dy = K.Device.of(rng.standard_normal((rows, dim)).astype(np.float32))
        w = K.Device.of(np.ones(dim, np.float32))
        out, dx, dw, db = K.Device(rows * dim * 4), K.Device(rows * dim * 4), K.Device(dim * 4), K.Device(dim * 4)
        ws = K.Device(lib.dllm_hip_layer_norm_backward_workspace(rows))
        t = timed(lambda: K.check(lib.dllm_hip_layer_norm(x.ptr, w.ptr, w.ptr, out.ptr, rows, dim, 1e-12, None)))
        report(f"layer_norm {rows}x{dim}", t, GBps=round(8 * rows * dim / t / 1e9, 1),
               hbm_frac=round(8 * rows * dim / t / hbm, 3))
        t = timed(lambda: K.check(lib.dllm_hip_layer_norm_backward(x.ptr, w.ptr, dy.ptr, dx.ptr, dw.ptr, db.ptr, rows,
                                                                   dim, 1e-12, ws.ptr, ws.nbytes, None)))
        report(f"layer_norm_backward {rows}x{dim}", t, GBps=round(12 * rows * dim / t / 1e9, 1),
               hbm_frac=round(12 * rows * dim / t / hbm, 3))
    for T, H, hd in [(512, 12, 64), (1024, 16, 64)]:
        qkv = K.Device.of(rng.standard_normal((T, H, hd)).astype(np.float32))
        bias = K.Device.of(rng.standard_normal((H, T, T)).astype(np.float32))
        out, dq, dk, dv = (K.Device(T * H * hd * 4) for _ in range(4))
        dbias, wts = K.Device(H * T * T * 4), K.Device(T * H * T * 4)
        ws = K.Device(lib.dllm_hip_biased_attention_backward_workspace(T, T, H, hd, hd))
        flop = 4.0 * T * T * H * hd
        t = timed(lambda: K.check(lib.dllm_hip_biased_attention(qkv.ptr, qkv.ptr, qkv.ptr, bias.ptr, out.ptr, T, T, H,
                                                                hd, hd, 0.125, ws.ptr, ws.nbytes, None)))
        report(f"biased_attention T={T} heads={H} head_dim={hd}", t, TFLOPs=round(flop / t / 1e12, 2))
        t = timed(lambda: K.check(lib.dllm_hip_biased_attention_weights(qkv.ptr, qkv.ptr, bias.ptr, wts.ptr, T, T, H,
                                                                        hd, 0.125, ws.ptr, ws.nbytes, None)))
        report(f"biased_attention_weights T={T} heads={H} head_dim={hd}", t, TFLOPs=round(flop / 2 / t / 1e12, 2))
        t = timed(lambda: K.check(lib.dllm_hip_biased_attention_backward(
            qkv.ptr, qkv.ptr, qkv.ptr, bias.ptr, qkv.ptr, dq.ptr, dk.ptr, dv.ptr, dbias.ptr, T, T, H, hd, hd, 0.125,
            ws.ptr, ws.nbytes, None)))
        report(f"biased_attention_backward T={T} heads={H} head_dim={hd}", t, TFLOPs=round(2 * flop / t / 1e12, 2))
    return 0


C2_SHAPES = dict(hidden=896, heads=14, kv_heads=2, head_dim=64, intermediate=4864, rope_theta=1e6)
C2_SWEEP = (1, 7, 64, 2048, 8192)


def c2_microbench(iters: int = 20) -> int:
    """the per-op backward kernels at Qwen2.5-0.5B layer shapes through the C ABI on
    device-resident inputs (weights N(0, 0.02), activations N(0, 1), upstream gradients N(0, 1e-3)), at each row count
    M of the sweep: the layer's seven linear_backward calls (dX and dW), dX and dW of the gate projection alone,
    rms_norm_backward, the RoPE backward of q and k, silu_backward over the SwiGLU width, causal GQA
    attention_backward over one sequence of M tokens, and one adamw_step over the layer's 14.9M parameters. Each op's
    time per call (mean of `iters` calls after 3 warmups) and its rate against the bound that applies: FP64 78.6
    TFLOP/s for the matmuls and attention, HBM 8 TB/s for the rest (plus the rate of the library's own device copy on
    this box, the practical streaming ceiling). One JSON line."""
    from etalii_dllm_amd import kernels as K

    lib, rng = K.lib, np.random.default_rng(0)
    H, nh, nkv, hd, inter = (C2_SHAPES[k] for k in ("hidden", "heads", "kv_heads", "head_dim", "intermediate"))
    hbm = 8.0e12

    def gauss(*shape, scale=1.0):
        return K.Device.of((rng.standard_normal(shape) * scale).astype(np.float32))

    def timed(run, n=iters) -> float:
        for _ in range(3):
            run()
        K.check(lib.dllm_hip_synchronize())
        t = time.perf_counter()
        for _ in range(n):
            run()
        K.check(lib.dllm_hip_synchronize())
        return (time.perf_counter() - t) / n

    ops = []

    def report(op, m, seconds, work, bound):
        rate = work / seconds
        if bound == "fp64":
            entry = {"op": op, "M": m, "us": round(seconds * 1e6, 2), "TFLOPs": round(rate / 1e12, 3),
                     "frac": round(rate / (FP64_PEAK_TFLOPS * 1e12), 4)}
        else:
            entry = {"op": op, "M": m, "us": round(seconds * 1e6, 2), "GBps": round(rate / 1e9, 1),
                     "frac": round(rate / hbm, 4)}
        ops.append(entry)
        log(json.dumps(entry))

    copy_bytes = 1 << 30
    src, dst = K.Device(copy_bytes), K.Device(copy_bytes)
    t_copy = timed(lambda: K.check(lib.dllm_hip_copy(dst.ptr, src.ptr, copy_bytes, None)), 10)
    copy_rate = 2.0 * copy_bytes / t_copy
    del src, dst
    mats = {"q": (H, nh * hd), "k": (H, nkv * hd), "v": (H, nkv * hd), "o": (nh * hd, H), "gate": (H, inter),
            "up": (H, inter), "down": (inter, H)}  # (in, out)
    weights = {n: gauss(o, i, scale=0.02) for n, (i, o) in mats.items()}
    mmax = C2_SWEEP[-1]
    x_in = {i: gauss(mmax, i) for i in {H, nh * hd, inter}}
    dy_out = {o: gauss(mmax, o, scale=1e-3) for o in {H, nh * hd, nkv * hd, inter}}
    dx = K.Device(mmax * max(H, inter, nh * hd) * 4)
    dw = K.Device(max(i * o for i, o in mats.values()) * 4)
    db = K.Device(max(o for _, o in mats.values()) * 4)
    norm_w = gauss(H, scale=0.02)
    qh, kh = gauss(mmax, nh, hd), gauss(mmax, nkv, hd)
    vh, douth = gauss(mmax, nkv, hd), gauss(mmax, nh, hd, scale=1e-3)
    gq, gk, gv = K.Device(mmax * nh * hd * 4), K.Device(mmax * nkv * hd * 4), K.Device(mmax * nkv * hd * 4)
    inv = np.ascontiguousarray(1.0 / (C2_SHAPES["rope_theta"] ** (np.arange(0, hd, 2, dtype=np.float64) / hd)))
    inv_d = K.Device.of(inv)
    pos_d = K.Device.of(np.arange(mmax, dtype=np.int64))
    n_params = sum(i * o for i, o in mats.values()) + 2 * H
    pp, gg = gauss(n_params, scale=0.02), gauss(n_params, scale=1e-3)
    mm, vv = gauss(n_params, scale=1e-4), K.Device.of(np.abs(rng.standard_normal(n_params) * 1e-6).astype(np.float32))
    for m in C2_SWEEP:
        n_it = iters if m >= 2048 else 5 * iters
        total, flop = 0.0, 0.0
        for name, (i, o) in mats.items():
            ws = K.Device(lib.dllm_hip_linear_backward_workspace(m, i, o))
            t = timed(lambda: K.check(lib.dllm_hip_linear_backward(x_in[i].ptr, weights[name].ptr, dy_out[o].ptr,
                                                                   dx.ptr, dw.ptr, None, m, i, o, ws.ptr, ws.nbytes,
                                                                   None)), n_it)
            total += t
            flop += 4.0 * m * i * o
        report("linear_backward (7 layer matrices, dX + dW)", m, total, flop, "fp64")
        i, o = mats["gate"]
        ws = K.Device(lib.dllm_hip_linear_backward_workspace(m, i, o))
        t = timed(lambda: K.check(lib.dllm_hip_linear_backward(x_in[i].ptr, weights["gate"].ptr, dy_out[o].ptr, dx.ptr,
                                                               None, None, m, i, o, ws.ptr, ws.nbytes, None)), n_it)
        report("dX gate (896 -> 4864)", m, t, 2.0 * m * i * o, "fp64")
        t = timed(lambda: K.check(lib.dllm_hip_linear_backward(x_in[i].ptr, weights["gate"].ptr, dy_out[o].ptr, None,
                                                               dw.ptr, db.ptr, m, i, o, ws.ptr, ws.nbytes, None)), n_it)
        report("dW + db gate (896 -> 4864)", m, t, 2.0 * m * i * o, "fp64")
        ws = K.Device(lib.dllm_hip_rms_norm_backward_workspace(m))
        t = timed(lambda: K.check(lib.dllm_hip_rms_norm_backward(x_in[H].ptr, norm_w.ptr, dy_out[H].ptr, dx.ptr,
                                                                 dw.ptr, m, H, 1e-6, 0, ws.ptr, ws.nbytes, None)), n_it)
        report("rms_norm_backward (dx, dw)", m, t, 12.0 * m * H, "hbm")
        wsq = K.Device(lib.dllm_hip_rope_workspace(m, hd))
        t = timed(lambda: (K.check(lib.dllm_hip_rope(qh.ptr, pos_d.ptr, inv_d.ptr, gq.ptr, m, nh, hd, hd, 0, 1,
                                                     wsq.ptr, wsq.nbytes, None)),
                           K.check(lib.dllm_hip_rope(kh.ptr, pos_d.ptr, inv_d.ptr, gk.ptr, m, nkv, hd, hd, 0, 1,
                                                     wsq.ptr, wsq.nbytes, None))), n_it)
        report("rope backward (q and k)", m, t, 8.0 * m * (nh + nkv) * hd, "hbm")
        t = timed(lambda: K.check(lib.dllm_hip_silu_backward(x_in[inter].ptr, dy_out[inter].ptr, dx.ptr, m * inter,
                                                             None)), n_it)
        report("silu_backward (SwiGLU width)", m, t, 12.0 * m * inter, "hbm")
        wsa = K.Device(lib.dllm_hip_attention_backward_workspace(m, m, nh, nkv, hd, hd, 1, 0, 0, 0.0))
        t = timed(lambda: K.check(lib.dllm_hip_attention_backward(
            qh.ptr, kh.ptr, vh.ptr, douth.ptr, gq.ptr, gk.ptr, gv.ptr, m, m, nh, nkv, hd, hd, 1.0 / np.sqrt(hd), 1, 0,
            0, 0.0, wsa.ptr, wsa.nbytes, None)), max(3, n_it // 4) if m >= 2048 else n_it)
        del wsa
        report("attention_backward (causal GQA 14/2 x 64)", m, t, 10.0 * hd * nh * m * (m + 1) / 2, "fp64")
    t = timed(lambda: K.check(lib.dllm_hip_adamw_step(pp.ptr, gg.ptr, mm.ptr, vv.ptr, n_params, 1e-4, 0.9, 0.999, 1e-8,
                                                      0.01, 0.1, 0.001, 1.0, None)))
    report("adamw_step (layer, 14.9M params)", n_params, t, 28.0 * n_params, "hbm")
    print(json.dumps({"metric": "C2 per-op backward microbench, Qwen2.5-0.5B layer shapes, bit-exact vs CPU",
                      "unit": "us per call", "higher_is_better": False, "n_gpus": 1, "dtype": "f64",
                      "data": "synthetic (Gaussian weights x 0.02, activations x 1, gradients x 1e-3)",
                      "config": {"workload": "Qwen2.5-0.5B layer backward ops", "M": list(C2_SWEEP), **C2_SHAPES},
                      "hbm_copy_GBps": round(copy_rate / 1e9, 1), "hbm_copy_frac": round(copy_rate / hbm, 4),
                      "ops": ops}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + ["c2"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-steps", type=int, default=None,
                    help="steps of the matmul-timing pass after the timed steps (default: --steps; 0 skips it)")
    ap.add_argument("--export-timing", action="store_true",
                    help="after the timed steps, time the model and checkpoint fingerprints streamed from device "
                         "memory (stderr only)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of 1 GiB (the reference kernel for HBM byte counters)")
    ap.add_argument("--traffic-summary", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV", "COPY_WRITE_CSV"),
                    help="turn rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE counter files into profiles/gemm_traffic.json")
    ap.add_argument("--kernels", action="store_true",
                    help="time the inference linear layers and encoder/T5 kernels instead of the step (one JSON line "
                         "per case)")
    args = ap.parse_args()
    if args.kernels:
        return kernel_suite()
    if args.config == "c2":
        return c2_microbench()
    if args.copy_calibration:
        return copy_calibration()
    if args.traffic_summary:
        return traffic_summary(args.config, *args.traffic_summary)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this backend runs the step on a single MI355X (got --gpus {args.gpus}); "
              "on more GPUs each would take whole windows, their gradients summed in window order", file=sys.stderr)
        return 2
    cfg = CONFIGS[args.config]
    from etalii_dllm_amd.kernels import check, lib
    from etalii_dllm_amd.trainer import Decoder, Trainer

    lib.dllm_hip_trainer_profile.argtypes = [C.c_void_p, C.c_int]
    lib.dllm_hip_trainer_profile_read.argtypes = [C.c_void_p, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                                                  C.POINTER(C.c_double)]
    decoder = Decoder(cfg["vocab"], cfg["hidden"], cfg["intermediate"], cfg["layers"], cfg["heads"], cfg["kv_heads"],
                      cfg["head_dim"], cfg["rms_norm_eps"], cfg["rope_theta"], cfg["tie_embeddings"],
                      cfg["attention_bias"], cfg.get("qk_norm", 0), 0, cfg.get("experts", 0),
                      cfg.get("experts_per_token", 0), cfg.get("normalize_expert_weights", False),
                      cfg.get("expert_intermediate", 0))
    lora = None
    if "lora" in cfg:
        from etalii_dllm_amd.trainer import lora_config

        lora = lora_config(cfg["lora"]["rank"], cfg["lora"]["alpha"], cfg["lora"]["targets"], base_quantize="q8_0")
    router_aux = cfg.get("router_aux_loss", 0.0)
    tokens_per_step = cfg["batch"] * cfg["seq"]
    log(f"creating trainer for {cfg['name']} ({tokens_per_step} tokens per step)")
    t0 = time.perf_counter()
    trainer = Trainer(decoder, tokens_per_step, cfg["batch"], cfg["seq"], lora=lora)
    init_weights(trainer, lib, tensor_shapes(cfg))
    if lora is not None:
        init_adapters(trainer, lib, cfg)
    log(f"weights ready in {time.perf_counter() - t0:.1f} s")
    roofline_steps = args.steps if args.roofline_steps is None else args.roofline_steps
    total = args.warmup + args.steps + roofline_steps
    windows = [make_windows(lib, cfg, s) for s in range(total)]
    for s in range(args.warmup):
        t1 = time.perf_counter()
        loss, norm = trainer.step(windows[s], LEARNING_RATE, s + 1, router_aux_loss=router_aux)
        log(f"warmup step {s + 1}: loss {loss:.6f} norm {norm:.6f} ({time.perf_counter() - t1:.2f} s)")
    # the timed steps: the step alone, nothing recorded around its launches
    check(lib.dllm_hip_synchronize())
    t0 = time.perf_counter()
    for s in range(args.warmup, args.warmup + args.steps):
        loss, norm = trainer.step(windows[s], LEARNING_RATE, s + 1, router_aux_loss=router_aux)
        log(f"step {s + 1}: loss {loss:.6f} norm {norm:.6f}")
    check(lib.dllm_hip_synchronize())
    elapsed = time.perf_counter() - t0
    # the matmul-timing steps: the same step with a pair of HIP events around every matmul launch on its stream
    # (the events add host and queue overhead to the step, so these steps are not the throughput figure)
    check(lib.dllm_hip_trainer_profile(trainer.handle, 1))
    t_roof = time.perf_counter()
    for s in range(args.warmup + args.steps, total):
        loss, norm = trainer.step(windows[s], LEARNING_RATE, s + 1, router_aux_loss=router_aux)
        log(f"matmul-timing step {s + 1}: loss {loss:.6f} norm {norm:.6f}")
    check(lib.dllm_hip_synchronize())
    roof_elapsed = time.perf_counter() - t_roof
    launches, ms, flops = C.c_int64(), C.c_double(), C.c_double()
    check(lib.dllm_hip_trainer_profile_read(trainer.handle, C.byref(launches), C.byref(ms), C.byref(flops)))
    check(lib.dllm_hip_trainer_profile(trainer.handle, 0))
    if args.export_timing:
        for kind, what in ((0, "model.dllm data"), (1, "checkpoint data")):
            t_start = time.perf_counter()
            digest = trainer.fingerprint(kind)
            seconds = time.perf_counter() - t_start
            log(f"{what} fingerprint {digest[:16]}...: {seconds:.2f} s")
    trainer.close()
    ms_per_step = elapsed * 1000.0 / args.steps
    achieved = flops.value / (ms.value * 1e9) if ms.value > 0 else None  # TFLOP/s
    if roofline_steps:
        log(f"matmuls: {launches.value} launches over {roofline_steps} steps, {ms.value:.1f} ms, {flops.value:.3e} "
            f"flop ({100.0 * ms.value / (roof_elapsed * 1000.0):.1f}% of those steps' time, "
            f"{roof_elapsed * 1000.0 / roofline_steps:.1f} ms per step with the events)")
    traffic = None
    traffic_file = ROOT / "profiles" / "gemm_traffic.json"
    if traffic_file.exists():
        entry = json.loads(traffic_file.read_text()).get(args.config)
        traffic = entry["bytes_per_launch"] if entry else None
    baseline = None
    if not args.no_cpu_baseline:
        log("timing the reference CPU path on a bounded sample")
        baseline = cpu_baseline(cfg)
    result = {
        "metric": METRIC if args.config == "c3" else f"finetune tokens/s, {cfg['name']} fp32 step, bit-exact vs CPU",
        "value": tokens_per_step * args.steps / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded Gaussian weights x 0.02, uniform random token ids)",
        "config": {"workload": f"{cfg['name']} " + ("LoRA step (forward, backward, adapter gradients, global-norm "
                                                     "clip, AdamW on the adapters)" if lora is not None else
                                                     "full fine-tune step (forward, backward, global-norm clip, AdamW)"),
                   "global_batch": cfg["batch"], "seq_len": cfg["seq"], "parallelism": "single GPU",
                   "layers": cfg["layers"], "hidden": cfg["hidden"], "vocab": cfg["vocab"]},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / FP64_PEAK_TFLOPS if achieved else None, "traffic": traffic,
                     "kernel": "gemm_mfma_kernel (FP64 MFMA matmul, every launch of the matmul-timing steps)",
                     "timing_steps": roofline_steps,
                     "step_fraction_of_peak": matmul_flops_per_step(cfg) / (ms_per_step * 1e9) / FP64_PEAK_TFLOPS},
        "cpu_baseline": baseline,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
