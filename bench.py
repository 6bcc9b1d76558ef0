#!/usr/bin/env python3
"""Benchmark of the Jevstral token loop on one MI355X.

Headline (the reference's own benchmark, `jev bench` prefill): a 256-token
causal prefill of the 26-layer Ministral-3 3B shape with Q8_0 weights, ending
in the final position's full-vocabulary logits.  value = prompt tokens per
second with the token ids and the model already resident in HBM.  Beside it,
the 4096-token-trunk, 9 x 48-token-branch tree decision (verdict rows only) in
ms per decision.

Weights are synthetic (N(0, 0.02) quantized to Q8_0 with the ggml reference
quantizer, norms 1.0) because no checkpoint is available offline; token ids are
uniform on the vocabulary.

One JSON line goes to stdout; progress goes to stderr.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm-shield_amd"))

PEAK_FP16_MFMA = 2.5e15  # dense fp16 MFMA, MI355X
PEAK_HBM = 8.0e12


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def prof_read(lib, h, cls):
    n = ctypes.c_int64()
    ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    rc = lib.jev_profile_read(h, cls, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by))
    assert rc == 0
    return n.value, ms.value, fl.value, by.value


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tree-steps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--no-tree", action="store_true", help="skip the tree-decision leg")
    ap.add_argument("--layers", type=int, default=26, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every config fits one MI355X)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import jev
    from jev import _lib as L

    cfg = jev.ModelConfig(n_layers=args.layers, initial_kv_capacity=4608)
    t0 = time.time()
    synth = jev.SynthModel(cfg, jev.TYPE_Q8_0)
    log(f"synthetic Q8_0 model generated in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = synth.open(0)
    lib = jev.lib()
    h = model.handle
    log(f"weights bound to HBM in {time.time() - t0:.1f}s")

    dev = torch.device("cuda:0")
    T = 256
    tokens = jev.random_tokens(T, cfg.vocab, 11)
    d_tok = torch.from_numpy(tokens.astype(np.int32)).to(dev)
    d_out = torch.empty(cfg.vocab, dtype=torch.float32, device=dev)

    def step():
        L.check(lib.jev_kv_reset(h))
        L.check(lib.jev_forward_device(h, ctypes.c_void_p(d_tok.data_ptr()), T, None, L.OUT_LAST_FULL, None, 0,
                                       ctypes.c_void_p(d_out.data_ptr())))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    L.check(lib.jev_profile_enable(h, 1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    L.check(lib.jev_sync(h))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gemm = prof_read(lib, h, L.PROF_GEMM)
    attn = prof_read(lib, h, L.PROF_ATTN)
    gemv = prof_read(lib, h, L.PROF_GEMV)
    L.check(lib.jev_profile_enable(h, 0))
    ms_step = elapsed / args.steps * 1e3
    tok_s = T * args.steps / elapsed
    log(f"prefill {T} tokens: {ms_step:.3f} ms/step, {tok_s:,.0f} tok/s")
    gpu_logits = d_out.cpu().numpy()

    gemm_avg_ms = gemm[1] / max(gemm[0], 1)
    gemm_tflops = gemm[2] / (gemm[1] * 1e-3) / 1e12 if gemm[1] > 0 else 0.0
    log(f"GEMM: {gemm[0]} launches, {gemm[1]:.2f} ms, {gemm_tflops:.1f} TFLOP/s algorithmic")
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_q8_0_prefill256_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")

    result = {
        "metric": "prefill tok/s @256 tok Q8_0 3B; ms per 4k-trunk 9-branch tree decision",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights, fp16x2 MFMA operands, fp32 accumulate",
        "data": "synthetic: N(0,0.02) weights quantized to Q8_0, norms 1.0, uniform token ids (seed 11)",
        "config": {"workload": "Ministral-3 3B shape (26 layers, d 3072, 32/8 heads x 128, ffn 9216, vocab 131072), "
                               "Q8_0, 256-token causal prefill + final-position full-vocab logits",
                   "global_batch": 1, "seq_len": T, "parallelism": "single GPU"},
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_q_kernel (Q8_0)",
            "achieved": round(gemm_tflops, 2),
            "peak": PEAK_FP16_MFMA / 1e12,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops * 1e12 / PEAK_FP16_MFMA, 4),
            "traffic": traffic,
            "launches": gemm[0] // args.steps,
            "avg_launch_us": round(gemm_avg_ms * 1e3, 2),
            "flops_per_launch": gemm[2] / max(gemm[0], 1),
            "alg_bytes_per_launch": round(gemm[3] / max(gemm[0], 1)),
        },
        "breakdown_ms_per_step": {
            "gemm": round(gemm[1] / args.steps, 4),
            "attention": round(attn[1] / args.steps, 4),
            "gemv_head": round(gemv[1] / args.steps, 4),
        },
    }

    # ---- tree decision (4096 trunk + 9 x 48 branches, verdict rows only)
    if not args.no_tree:
        trunk_n, nb, bl = 4096, 9, 48
        toks = jev.random_tokens(trunk_n + nb * bl, cfg.vocab, 23)
        offsets = [trunk_n + b * bl for b in range(nb)]
        lay = jev.TokenLayout.tree(0, trunk_n, offsets, trunk_n + nb * bl)
        lay_c = lay.to_c()
        rows = np.array([jev.VERDICT_YES, jev.VERDICT_NO], np.int32)
        d_tt = torch.from_numpy(toks).to(dev)
        d_v = torch.empty(nb * 2, dtype=torch.float32, device=dev)

        def decide():
            L.check(lib.jev_kv_reset(h))
            L.check(lib.jev_forward_device(h, ctypes.c_void_p(d_tt.data_ptr()), len(toks), ctypes.byref(lay_c),
                                           L.OUT_SELECTED, rows.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), 2,
                                           ctypes.c_void_p(d_v.data_ptr())))

        decide()
        torch.cuda.synchronize()
        L.check(lib.jev_profile_enable(h, 1))
        t0 = time.perf_counter()
        for _ in range(args.tree_steps):
            decide()
        L.check(lib.jev_sync(h))
        torch.cuda.synchronize()
        tree_ms = (time.perf_counter() - t0) / args.tree_steps * 1e3
        tg = prof_read(lib, h, L.PROF_GEMM)
        ta = prof_read(lib, h, L.PROF_ATTN)
        L.check(lib.jev_profile_enable(h, 0))
        v = d_v.cpu().numpy().reshape(nb, 2)
        z = v[:, 0] - v[:, 1]
        log(f"tree decision: {tree_ms:.2f} ms; gemm {tg[1] / args.tree_steps:.2f} ms, attention {ta[1] / args.tree_steps:.2f} ms")
        result["tree_decision_ms"] = round(tree_ms, 3)
        result["tree_breakdown_ms"] = {
            "gemm": round(tg[1] / args.tree_steps, 3),
            "gemm_tflops": round(tg[2] / (tg[1] * 1e-3) / 1e12, 2) if tg[1] else None,
            "attention": round(ta[1] / args.tree_steps, 3),
            "attention_tflops": round(ta[2] / (ta[1] * 1e-3) / 1e12, 2) if ta[1] else None,
        }
        result["tree_z"] = [round(float(x), 5) for x in z]

    # ---- CPU baseline: the oracle on the host cores, one 256-token prefill
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        from oracle import oracle

        threads = max(1, min(16, os.cpu_count() or 1))
        oracle.set_threads(threads)
        ref = oracle.OracleModel(cfg).bind_synth(synth)
        t0 = time.perf_counter()
        cpu_logits = ref.forward(tokens)
        cpu_s = time.perf_counter() - t0
        err = float(np.max(np.abs(gpu_logits - cpu_logits) / np.maximum(1.0, np.abs(cpu_logits))))
        log(f"CPU oracle: {cpu_s:.2f}s for the 256-token prefill ({threads} threads); GPU vs CPU logits worst {err:.2e}")
        result["cpu_baseline"] = {
            "value": round(T / cpu_s, 2),
            "unit": "tok/s",
            "cores": threads,
            "kind": "port",
            "sample": "one full 256-token Q8_0 prefill + final-position full-vocab logits of the same 26-layer "
                      "synthetic model (C restatement of the reference's managed Float path)",
        }
        result["parity_logits_worst_rel"] = err
        ref.close()

    model.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
