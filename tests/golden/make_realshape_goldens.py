"""Writes tests/golden/realshape_<name>.json: the oracle's training steps over the reference's own kernels
(oracle/_ref/libdllm_ref.so, compiled from the reference headers by oracle/Makefile) at the real-shape configurations
of tests/realshape.py, recorded as SHA-256 digests of every gradient, parameter and AdamW moment after each step,
plus the loss and gradient norm as exact hex doubles.

Run from the repository root, in the container that holds the reference checkout (minutes per configuration; the
reference's head matmul, cross-entropy, attention backward and AdamW dominate):
    python tests/golden/make_realshape_goldens.py c1 c3 c4 c5
"""

from __future__ import annotations

import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import oracle_lib as O  # noqa: E402
import realshape as R  # noqa: E402


def dense_run(cfg: R.RealShape, kern) -> dict:
    d = cfg.decoder
    params = R.weights(cfg)
    record = {"inputs": R.digest(O.concatenated(params))}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=cfg.learning_rate, schedule="constant")
    windows = R.windows(cfg)
    steps = []
    for step in range(1, cfg.steps + 1):
        t0 = time.time()
        loss, _, norm, grads = O.train_step(kern, d, params, m, v, windows, opt, step, cfg.steps,
                                            router_aux_loss=cfg.router_aux_loss)
        tensors = {name: {"grad": R.digest(grads[name]), "param": R.digest(params[name]), "m": R.digest(m[name]),
                          "v": R.digest(v[name])} for name in O.tensor_order(d.tensor_shapes())}
        steps.append({"loss": R.double_hex(loss), "norm": R.double_hex(norm), "tensors": tensors})
        print(f"{cfg.name} step {step}: loss {loss!r} norm {norm!r} ({time.time() - t0:.0f} s)", flush=True)
    record["steps"] = steps
    return record


def lora_run(cfg: R.RealShape, kern) -> dict:
    d = cfg.decoder
    base = R.weights(cfg)
    adapters = R.adapters(cfg)
    record = {"inputs": R.digest(O.concatenated(base)), "adapter_inputs": R.digest(O.concatenated(adapters))}
    if cfg.base_quantize == "q8_0":
        base = R.quantized_base(cfg, base, O.ref().ref_quantize_q8_0)
    m = {n: np.zeros_like(a) for n, a in adapters.items()}
    v = {n: np.zeros_like(a) for n, a in adapters.items()}
    opt = O.AdamWConfig(learning_rate=cfg.learning_rate, schedule="constant")
    windows = R.windows(cfg)
    targets = O.lora_target_weights(d, cfg.lora)
    steps = []
    for step in range(1, cfg.steps + 1):
        t0 = time.time()
        out: dict = {}
        loss, norm = O.lora_train_step(kern, d, base, adapters, m, v, windows, opt, step, cfg.steps, cfg.lora,
                                       router_aux_loss=cfg.router_aux_loss, out=out)
        tensors = {name: {"grad": R.digest(out["adapter_grads"][name]), "param": R.digest(adapters[name]),
                          "m": R.digest(m[name]), "v": R.digest(v[name])} for name in O.tensor_order(adapters)}
        for name in targets:  # the merged weights' gradients (what the adapters' gradients are formed from)
            tensors[name] = {"grad": R.digest(out["weight_grads"][name])}
        steps.append({"loss": R.double_hex(loss), "norm": R.double_hex(norm), "tensors": tensors})
        print(f"{cfg.name} step {step}: loss {loss!r} norm {norm!r} ({time.time() - t0:.0f} s)", flush=True)
    record["steps"] = steps
    return record


def main(names: list[str]) -> None:
    if not O.reference_available():
        raise SystemExit("oracle/_ref/libdllm_ref.so is not built (make -C oracle, with the reference checkout)")
    O.ref().ref_set_threads(C.c_size_t(os.cpu_count() or 1))
    kern = O.ref_kernels()
    for name in names:
        cfg = R.CONFIGS[name]
        t0 = time.time()
        record = lora_run(cfg, kern) if cfg.lora is not None else dense_run(cfg, kern)
        record = {"config": name, "notes": cfg.notes, "checker": "oracle step orchestration over oracle/_ref",
                  **record}
        (HERE / f"realshape_{name}.json").write_text(json.dumps(record, indent=1, sort_keys=True) + "\n")
        print(f"{name}: {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or sorted(R.CONFIGS))
