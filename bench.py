"""Benchmark of the GPT-2 token loop on one MI355X.

Default workload (BASELINE.json metric "decode tokens/s (GPT-2 small b=1) +
achieved HBM GB/s as % of peak"): configuration c1 = GPT-2 small, fp32,
random-init N(0, 0.02) weights from seed 1234, batch 1, prompt of 32 uniform
random ids, greedy decode of 64 tokens (1 prefill + 63 decode steps).

One "step" is one such generate_cached job on weights already resident in
HBM. `value` = decode tokens/s over the timed steps (decode time measured with
HIP events on the library's stream); prefill is reported separately.
Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode tokens/s (GPT-2 small b=1) + achieved HBM GB/s as % of peak"

WORKLOADS = {
    # name: (shape, batch, prompt, new tokens, storage)
    "c1": ("small", 1, 32, 64, "f32"),
    "c2": ("small", 8, 128, 256, "f32"),
    "c3": ("medium", 1, 512, 512, "f32"),
    "c5": ("xl", 16, 64, 256, "bf16"),
}


def decode_bytes(sh, B, past, wbytes):
    """Algorithmic HBM bytes of one decode step at past length `past`:
    weights once, KV read for past+1 positions plus the new row written,
    embedding rows read, logits written."""
    L, d, V = sh.n_layer, sh.n_embd, sh.vocab_size
    weights = (L * (12 * d * d + 13 * d) + V * d + 2 * d)
    # matrices and wte in storage type, LN/bias in f32
    mats = L * 12 * d * d + V * d
    wb = mats * wbytes + (weights - mats) * 4
    kv = B * L * 2 * d * 4 * (past + 2)
    emb = B * 2 * d * 4
    return wb + kv + emb + B * V * 4


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_oracle(m, O, prompt, n_decode):
    """(prefill seconds, decode seconds) of one greedy run on a fresh cache."""
    c = m.new_cache()
    t0 = time.perf_counter()
    lg = m.forward_cached(prompt, c)
    t1 = time.perf_counter()
    tok = O.argmax(lg[-1])
    for _ in range(n_decode):
        lg = m.forward_cached([tok], c)
        tok = O.argmax(lg[0])
    return t1 - t0, time.perf_counter() - t1


# The CPU baseline's bounded sample per workload (BASELINE.md plans subsets
# for the slow configurations): (prompt tokens timed, decode steps timed,
# what the sample stands for). The reference runs one sequence at a time, so
# a batch of B runs B such samples one after another: its tokens/s is the
# single-sequence rate.
CPU_SAMPLES = {
    "c1": (32, 24, "c1's prompt of 32 then 24 of its 63 decode steps"),
    "c2": (128, 16, "one of c2's 8 sequences: its prompt of 128 then 16 of its 255 decode steps"),
    "c3": (128, 16, "c3's model: a prompt of 128 (of 512) then 16 decode steps"),
    "c5": (64, 8, "one of c5's 16 sequences: its prompt of 64 then 8 of its 255 decode steps"),
    "c4": (128, 0, "one of c4's 32 sequences, its first 128 of 1024 tokens (prefill only)"),
}


def cpu_baseline(sd, sh, prompt, n_decode, all_threads, what):
    """Time the CPU oracle (a C restatement of gpt2.rs, built -O3 for
    x86-64-v3, the tied LM head multiplying a transpose materialised per call
    as gpt2.rs:395 does) on a bounded sample: with 1 thread, as the
    reference's single-threaded ndarray GEMM (the reported value), and with
    all_threads GEMM threads beside it."""
    from oracle import oracle as O
    O.build()
    m = O.OracleModel.from_shape(sd, sh, threads=1, lm_direct=False)
    pre, dec = _time_oracle(m, O, prompt, n_decode)
    rate = (n_decode / dec) if n_decode else len(prompt) / pre
    out = {"value": rate, "unit": "tokens/s", "cores": 1, "kind": "port",
           "sample": f"{what}: prefill {pre * 1e3:.0f} ms" + (f", {n_decode} greedy decode steps {dec * 1e3:.0f} ms"
                                                              if n_decode else "")
                     + "; oracle/gpt2_oracle.c (C restatement of gpt2.rs), 1 thread",
           "prefill_tok_s": len(prompt) / pre, "cpu": _cpu_model(), "nproc": os.cpu_count()}
    if all_threads > 1:
        m.set_threads(all_threads)
        pre, dec = _time_oracle(m, O, prompt, n_decode)
        out["all_cores"] = {"threads": all_threads, "value": (n_decode / dec) if n_decode else len(prompt) / pre,
                            "prefill_tok_s": len(prompt) / pre}
    return out


MFMA_FP32_PEAK_TFLOPS = 157.3
# dense bf16 MFMA peak; a GEMM with bf16 weights runs each f32 product as
# three exact bf16 MFMA products (the activation split into three bf16
# parts), so its peak in f32 flops is a third of it
MFMA_BF16_PEAK_TFLOPS = 2500.0
BF16X3_PEAK_TFLOPS = MFMA_BF16_PEAK_TFLOPS / 3
PREFILL_WORKLOADS = {
    # name: (shape, batch, tokens): forward_cached on an empty cache, full [T, V] logits per sequence
    "c4": ("large", 32, 1024),
}


def prefill_flops(sh, B, T):
    """Algorithmic flops of forward_cached over T new tokens on an empty
    cache: the four Conv1D GEMMs, causal QK^T and PV, and the LM head over
    every row (the reference computes [T, V] logits)."""
    L, d, V = sh.n_layer, sh.n_embd, sh.vocab_size
    return B * (2 * T * 12 * d * d * L + 4 * d * L * T * (T + 1) // 2 + 2 * T * d * V)


def run_prefill(a):
    from rusttorch_amd import synth
    from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Model

    shape_name, B, T = PREFILL_WORKLOADS[a.workload]
    sh = synth.SHAPES[shape_name]
    sd = synth.make_weights(sh)
    cfg = Gpt2Config(sh.vocab_size, sh.n_positions, sh.n_embd, sh.n_layer, sh.n_head, sh.layer_norm_epsilon)
    m = Gpt2Model.from_state_dict(sd, cfg)
    ids = np.stack([synth.make_tokens(T, sh.vocab_size, stream=b) for b in range(B)])
    cache = m.new_cache(B)
    print("[bench] model resident; warming up", file=sys.stderr, flush=True)
    for _ in range(a.warmup):
        cache.clear()
        m.forward_cached_batched(ids, cache, want_logits=False)
    times = []
    for _ in range(a.steps):
        cache.clear()
        t0 = time.perf_counter()
        m.forward_cached_batched(ids, cache, want_logits=False)  # logits stay in HBM
        times.append(time.perf_counter() - t0)
    print("[bench] timed steps done", file=sys.stderr, flush=True)
    del m
    step_s = float(np.mean(times))
    flops = prefill_flops(sh, B, T)
    achieved = flops / step_s / 1e12
    out = {
        "metric": f"prefill tokens/s (GPT-2 {shape_name} b={B}, {T} tokens)",
        "value": round(B * T / step_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,0.02) random-init weights, uniform random token ids",
        "config": {"workload": f"{a.workload}: GPT-2 {shape_name}, batch {B}, prefill {T} tokens, full logits",
                   "batch": B, "tokens": T, "weights": "f32"},
        "roofline": {"bound": "mfma", "kernel": "whole prefill (gemm_lds_kernel dominant)",
                     "achieved": round(achieved, 2), "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4), "flops_per_step": flops,
                     "traffic": None},
    }
    if not a.no_cpu:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        n_cpu, _, what = CPU_SAMPLES[a.workload]
        out["cpu_baseline"] = cpu_baseline(sd, sh, ids[0, :n_cpu], 0, a.cpu_threads, what)
    print(json.dumps(out))


def measured_traffic(workload, persistent):
    """HBM bytes per decode step measured by the rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes summarised in profiles/ (scaled by the copy-kernel
    calibration recorded there): per decode_step_kernel launch at batch 1,
    summed over the kernels of one step of the batched graph otherwise; None
    when no summary exists."""
    name = f"decode_step_kernel_{workload}" if persistent else f"decode_step_graph_{workload}"
    path = os.path.join(ROOT, "profiles", f"{name}_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:") or line.startswith("traffic_bytes_per_step:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def prefill_bytes(sh, B, T, wbytes):
    """Algorithmic HBM bytes of forward_cached over T tokens on an empty
    cache: weights once, the T embedding rows, the K/V rows written and every
    row's logits written (the reference computes [T, V])."""
    L, d, V = sh.n_layer, sh.n_embd, sh.vocab_size
    weights = (L * (12 * d * d + 13 * d) + V * d + 2 * d)
    mats = L * 12 * d * d + V * d
    wb = mats * wbytes + (weights - mats) * 4
    return wb + B * T * (2 * d * wbytes + L * 2 * d * 4 + V * 4)


def prefill_roofline(sh, B, T, wbytes, ms):
    """Roofline of the prefill leg: HBM when its arithmetic intensity is
    below the MFMA ridge (peak / 8 TB/s), MFMA otherwise. The peak is fp32
    MFMA for f32 weights; for bf16 weights the GEMMs run on bf16 MFMA with
    three exact products per f32 product (mfma "bf16x3"), so the peak in
    algorithmic f32 flops is the dense bf16 peak / 3."""
    flops = prefill_flops(sh, B, T)
    nbytes = prefill_bytes(sh, B, T, wbytes)
    s = ms / 1e3
    bf16 = wbytes == 2
    peak = BF16X3_PEAK_TFLOPS if bf16 else MFMA_FP32_PEAK_TFLOPS
    if flops / nbytes < peak * 1e12 / (HBM_PEAK_GBS * 1e9):
        ach = nbytes / s / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "bytes": int(nbytes), "ms": round(ms, 4)}
    ach = flops / s / 1e12
    return {"bound": "mfma", "mfma": "bf16x3" if bf16 else "fp32", "achieved": round(ach, 2),
            "peak": round(peak, 1), "unit": "TFLOP/s", "frac": round(ach / peak, 4), "flops": int(flops),
            "ms": round(ms, 4)}


def calib_copy(nbytes):
    """One hipMemset (a fill kernel writing nbytes) and one device-to-device
    hipMemcpy (the runtime's copy kernel: reads and writes nbytes), so that a
    rocprofv3 --pmc pass over this run can scale FETCH_SIZE / WRITE_SIZE."""
    import ctypes as C
    try:
        hip = C.CDLL("libamdhip64.so")
    except OSError:
        hip = C.CDLL("/opt/rocm/lib/libamdhip64.so")
    src, dst = C.c_void_p(), C.c_void_p()
    n = C.c_size_t(nbytes)
    ok = hip.hipMalloc(C.byref(src), n) == 0 and hip.hipMalloc(C.byref(dst), n) == 0
    ok = ok and hip.hipMemset(src, 1, n) == 0 and hip.hipDeviceSynchronize() == 0
    ok = ok and hip.hipMemcpy(dst, src, n, 3) == 0 and hip.hipDeviceSynchronize() == 0  # 3: device to device
    for p in (src, dst):
        if p.value:
            hip.hipFree(p)
    if not ok:
        raise RuntimeError("calibration copy failed")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c1", choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS))
    ap.add_argument("--cpu-decode-steps", type=int, default=24)
    # a GPU box gives one GPU a 16-core CPU share, whatever os.cpu_count() says
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1),
                    help="GEMM threads of the all-cores CPU variant (the reported value uses 1)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one device-to-device copy of 256 MiB (untimed): the reference kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "sharding is described in DESIGN.md, not run", file=sys.stderr)
        sys.exit(2)

    if a.workload in PREFILL_WORKLOADS:
        run_prefill(a)
        return

    from rusttorch_amd import synth
    from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Model

    shape_name, B, n_prompt, n_new, storage = WORKLOADS[a.workload]
    sh = synth.SHAPES[shape_name]
    t = time.perf_counter()
    sd = synth.make_weights(sh, bf16=(storage == "bf16"))
    print(f"[bench] weights generated in {time.perf_counter() - t:.1f}s", file=sys.stderr, flush=True)
    cfg = Gpt2Config(sh.vocab_size, sh.n_positions, sh.n_embd, sh.n_layer, sh.n_head, sh.layer_norm_epsilon)
    m = Gpt2Model.from_state_dict(sd, cfg, storage=storage)
    prompts = np.stack([synth.make_tokens(n_prompt, sh.vocab_size, stream=b) for b in range(B)])
    if a.calib_copy:
        calib_copy(256 << 20)
    print("[bench] model resident; warming up", file=sys.stderr, flush=True)
    for _ in range(a.warmup):
        m.generate_cached_batched(prompts, n_new)
    t0 = time.perf_counter()
    tims = []
    ids = None
    for _ in range(a.steps):
        ids, tm = m.generate_cached_batched(prompts, n_new, timing=True)
        tims.append(tm)
    wall = time.perf_counter() - t0
    print("[bench] timed steps done", file=sys.stderr, flush=True)

    dec_ms = sum(t["decode_ms"] for t in tims)
    pre_ms = sum(t["prefill_ms"] for t in tims)
    dec_steps = sum(t["decode_steps"] for t in tims)
    dec_tok_s = B * dec_steps / (dec_ms / 1e3)
    wbytes = 2 if storage == "bf16" else 4
    step_bytes = [decode_bytes(sh, B, n_prompt + i, wbytes) for i in range(n_new - 1)]
    avg_bytes = float(np.mean(step_bytes))
    step_ms = dec_ms / dec_steps
    # The decode step's average duration over the timed region: HIP events on
    # the library's stream bracket each job's back-to-back decode launches
    # (one persistent decode_step_kernel launch per token at batch 1, one
    # replay of the per-op step graph otherwise), so this includes the gaps
    # between launches and never less than the kernels themselves.
    persistent = B == 1
    if persistent:
        kernel = "decode_step_kernel (persistent, one launch per decode step)"
    else:
        kernel = "decode step (graph of per-op kernels: tile-ordered GEMVs, fused attention)"
    dur_ms = step_ms
    achieved = avg_bytes / (dur_ms / 1e3) / 1e9
    traffic = measured_traffic(a.workload, persistent)
    out = {
        "metric": METRIC,
        "value": round(dec_tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(wall / a.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if storage == "f32" else "f32 (bf16 weights)",
        "data": "synthetic: seeded N(0,0.02) random-init weights, uniform random token ids",
        "config": {"workload": f"{a.workload}: GPT-2 {shape_name}, batch {B}, prompt {n_prompt}, greedy {n_new}",
                   "batch": B, "prompt": n_prompt, "new_tokens": n_new, "weights": storage},
        "prefill_tok_s": round(B * n_prompt * a.steps / (pre_ms / 1e3), 1),
        "prefill_roofline": prefill_roofline(sh, B, n_prompt, wbytes, pre_ms / a.steps),
        "decode_ms_per_token_step": round(step_ms, 4),
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": int(avg_bytes), "avg_launch_ms": round(dur_ms, 5), "traffic": traffic},
        "first_ids": ids[0, n_prompt:n_prompt + 8].tolist(),
    }
    if not a.no_cpu:
        print("[bench] timing the CPU oracle sample", file=sys.stderr, flush=True)
        del m
        n_cpu, n_dec, what = CPU_SAMPLES[a.workload]
        if a.workload == "c1":
            n_dec = a.cpu_decode_steps
        out["cpu_baseline"] = cpu_baseline(sd, sh, prompts[0, :n_cpu], n_dec, a.cpu_threads, what)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
