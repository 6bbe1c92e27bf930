"""End-to-end prefill / decode latency of a Llama-shaped model whose attention
runs on libaoakv.so, with the reference latency driver's CSV row
(latency/bench_latency.py:42-200): the method, the md5 of the library that
was loaded, GPU, model, context, budget, page size, mean and std of the
prefill time and of the per-token decode time.

    python -m aoakv.latency --kernel aoa_kv --model longchat-7b-v1.5-32k \\
        --context_len 8192 --decode_len 256 --token_budget 1024 --out results.csv

``--kernel`` picks the tree as the reference driver's flag does
(bench_latency.py:27-32,49-64): ``aoa_kv`` is the value-aware score (CSV
method AOA_KV), ``quest_orig`` the plain Quest bound (method QUEST); both
run on libaoakv.so -- the package's own build, or the one the environment
variable AOAKV_LIB names -- and the md5 of the library loaded goes into every
row.  ``--method`` is the older spelling of the same choice.  Both use the
simulation's selection unless ``--semantics quest_kernel`` asks for the
reference kernels' convention.  ``--graph`` replays each decode step's
layers from a HIP graph (``QuestLlamaModel.decode_graphed``): at batch 1 the
eager step is bound by its per-layer host dispatch.  Weights are random and
seeded (no checkpoint is loaded; latency does not depend on weight values),
inputs are random
embeddings as in the reference driver, and timing uses events with a
synchronize on both sides after ``--warmup`` discarded iterations.  The
decode workspace's error word is read once per iteration (every step with
``--debug_checks``); a flagged error ends the run.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import time
from pathlib import Path

KERNELS = {"aoa_kv": "AOA_KV", "quest_orig": "QUEST"}   # tree -> CSV method label

CSV_FIELDS = [
    "method", "kernel_md5", "gpu", "model", "context_len", "token_budget",
    "page_size", "decode_len", "iteration", "prefill_ms", "prefill_std_ms",
    "decode_ms_per_token", "decode_std_ms", "timestamp",
]


def parse_args(argv=None):
    from .shim import MODEL_SHAPES
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--kernel", choices=sorted(KERNELS), default=None,
                   help="which tree to measure: aoa_kv (value-aware) or quest_orig (plain Quest)")
    p.add_argument("--method", choices=sorted(KERNELS.values()), default=None,
                   help="the same choice by CSV label (AOA_KV / QUEST)")
    p.add_argument("--debug_checks", action="store_true",
                   help="read the decode workspace error word after every decode step "
                        "(synchronizes; off: once per iteration)")
    p.add_argument("--semantics", choices=["sim", "quest_kernel"], default="sim")
    p.add_argument("--model", choices=sorted(MODEL_SHAPES), default="longchat-7b-v1.5-32k")
    p.add_argument("--layers", type=int, default=None,
                   help="override the layer count (a shorter stack for smoke runs)")
    p.add_argument("--context_len", type=int, default=8192)
    p.add_argument("--decode_len", type=int, default=256)
    p.add_argument("--token_budget", type=int, default=1024)
    p.add_argument("--page_size", type=int, default=16)
    p.add_argument("--iteration", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--roctx", action="store_true",
                   help="open the reference's nvtx ranges as roctx ranges (aoakv.tracing; "
                        "recorded by rocprofv3 --marker-trace)")
    p.add_argument("--three_call", action="store_true",
                   help="decode with the reference's three calls instead of one launch")
    p.add_argument("--graph", action="store_true",
                   help="replay each decode step's layers from a HIP graph (the host planner "
                        "runs eagerly before each replay; CSV method gets a _graph suffix)")
    p.add_argument("--out", default=None, help="CSV to append to (optional)")
    args = p.parse_args(argv)
    if args.kernel and args.method and KERNELS[args.kernel] != args.method:
        p.error(f"--kernel {args.kernel} and --method {args.method} disagree")
    args.method = KERNELS[args.kernel] if args.kernel else (args.method or "AOA_KV")
    if args.graph and args.debug_checks:
        p.error("--debug_checks synchronizes after every step; it cannot run inside --graph")
    return args


def main(argv=None):
    args = parse_args(argv)
    import numpy as np
    import torch

    from . import _lib
    from .shim import MODEL_SHAPES, QuestLlamaModel

    if args.roctx:
        from . import tracing
        tracing.enable()
    lib_path = Path(_lib.loaded_path()).resolve()
    md5 = hashlib.md5(lib_path.read_bytes()).hexdigest()
    device = torch.device("cuda:0")
    dtype = torch.float16
    gpu = torch.cuda.get_device_name(0)
    cfg = MODEL_SHAPES[args.model]
    if args.layers is not None:
        cfg = type(cfg)(**{**cfg.__dict__, "num_hidden_layers": args.layers})
    print(f"libaoakv.so : {lib_path}\nmd5         : {md5}\ngpu         : {gpu}\n"
          f"model       : {args.model} ({cfg.num_hidden_layers} layers, random weights)",
          flush=True)

    torch.set_default_dtype(dtype)
    with device:
        model = QuestLlamaModel(cfg, single_launch=not args.three_call).random_init(0)
    torch.set_default_dtype(torch.float32)
    model.quest_init(page_size=args.page_size,
                     max_seq_len=args.context_len + args.decode_len + 512,
                     token_budget=args.token_budget, dtype=dtype, device=device,
                     value_aware=args.method == "AOA_KV", semantics=args.semantics)

    prefill_ms, decode_ms = [], []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g = torch.Generator(device=device).manual_seed(1)
    with torch.inference_mode():
        for it in range(args.warmup + args.iteration):
            measured = it >= args.warmup
            x = torch.randn(1, args.context_len, cfg.hidden_size, generator=g, dtype=dtype,
                            device=device)
            torch.cuda.synchronize()
            start.record()
            model(x)
            end.record()
            torch.cuda.synchronize()
            if measured:
                prefill_ms.append(start.elapsed_time(end))
            for _ in range(args.decode_len):
                x = torch.randn(1, 1, cfg.hidden_size, generator=g, dtype=dtype, device=device)
                torch.cuda.synchronize()
                start.record()
                model.decode_graphed(x) if args.graph else model(x)
                end.record()
                torch.cuda.synchronize()
                if measured:
                    decode_ms.append(start.elapsed_time(end))
                if args.debug_checks:
                    model.iController.check_errors()
            model.iController.check_errors()  # once per iteration (raises on a flagged error)
            model.quest_clear()
            print(f"iteration {it} done ({'measured' if measured else 'warmup'})", flush=True)

    row = {
        "method": (args.method + ("" if args.semantics == "sim" else "_quest_kernel") +
                   ("_graph" if args.graph else "")),
        "kernel_md5": md5, "gpu": gpu, "model": args.model, "context_len": args.context_len,
        "token_budget": args.token_budget, "page_size": args.page_size,
        "decode_len": args.decode_len, "iteration": args.iteration,
        "prefill_ms": round(float(np.mean(prefill_ms)), 3),
        "prefill_std_ms": round(float(np.std(prefill_ms)), 3),
        "decode_ms_per_token": round(float(np.mean(decode_ms)), 4),
        "decode_std_ms": round(float(np.std(decode_ms)), 4),
        "timestamp": time.strftime("%Y-%m-%dT%H:%M:%S"),
    }
    print(",".join(CSV_FIELDS))
    print(",".join(str(row[k]) for k in CSV_FIELDS))
    if args.out:
        out = Path(args.out)
        out.parent.mkdir(parents=True, exist_ok=True)
        new = not out.exists()
        with out.open("a", newline="") as f:
            w = csv.DictWriter(f, fieldnames=CSV_FIELDS)
            if new:
                w.writeheader()
            w.writerow(row)
        print(f"appended to {out}")
    return row


if __name__ == "__main__":
    main()
