"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline metric "Q8_0 matvec HBM GB/s (% peak)": a step is one bs=1
pass of the Q8_0 matvec over the Qwen2.5-1.5B projection shapes
(N x K) 1536x1536 (q/o), 256x1536 (k/v), 8960x1536 gate+up as one fused
launch, 1536x8960 (down) and 151936x1536 (lm_head), weights resident in HBM.
Weight copies rotate so that each step streams from HBM rather than the
256 MB Infinity Cache. value = algorithmic bytes (weights + int8 activations
with f32 scales + f32 outputs) of the timed steps / timed wall time.

Prints one JSON line (see the repository's driver contract).
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "uefi-gpu_amd"))

import numpy as np  # noqa: E402

import uq  # noqa: E402

METRIC = "Q8_0 matvec HBM GB/s (% peak); bs=1 decode tok/s, Qwen2.5-1.5B shape"
HBM_PEAK_GBS = 8000.0
# HBM bytes per lm_head launch (151936x1536 Q8_0), from rocprofv3 PMC passes
# over this script: FETCH_SIZE 121,106.8 KiB x 1.99993 + WRITE_SIZE 593.5 KiB x 1.0,
# factors from 1 GiB read/copy probe kernels in the same runs
# (profiles/q8_matvec_lm_head_pmc.md).
LM_HEAD_TRAFFIC_BYTES = 248_626_178

# (name, N rows, K, fused pair)
SHAPES = [("attn_q/o", 1536, 1536, False), ("attn_k/v", 256, 1536, False),
          ("ffn_gate+up", 8960, 1536, True), ("ffn_down", 1536, 8960, False),
          ("lm_head", 151936, 1536, False)]


def q8_bytes(N, K):
    """Algorithmic bytes of one Q8_0 matvec: weights + int8 x + f32 scales + f32 y."""
    return N * (K // 32) * 34 + K + (K // 32) * 4 + 4 * N


# AMD x86 family numbers of the server cores (AMD's published family/model
# assignments): 0x17 Zen/Zen 2, 0x19 Zen 3/Zen 4, 0x1A Zen 5
AMD_FAMILIES = {0x17: {(0x00, 0x2F): "Zen / Zen+ (EPYC 7001)", (0x30, 0x3F): "Zen 2 (EPYC 7002, Rome)"},
                0x19: {(0x00, 0x0F): "Zen 3 (EPYC 7003, Milan)", (0x10, 0x1F): "Zen 4 (EPYC 9004, Genoa)",
                       (0xA0, 0xAF): "Zen 4c (EPYC 9004, Bergamo)"},
                0x1A: {(0x00, 0x1F): "Zen 5 (EPYC 9005, Turin)"}}


def cpu_model():
    """The first core's model string from /proc/cpuinfo with its x86 family,
    model and stepping (a VM may report only a generic name such as "AMD
    EPYC"; family/model still identify the core), the L3-visible cache size
    and the clock the kernel reports."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, v = line.partition(":")
            fields[k.strip()] = v.strip()
    except OSError:
        return platform.processor()
    name = fields.get("model name", platform.processor())
    try:
        fam, mod, step = int(fields["cpu family"]), int(fields["model"]), int(fields["stepping"])
    except (KeyError, ValueError):
        return name
    out = "%s (family 0x%X model 0x%X stepping %d" % (name, fam, mod, step)
    for (lo, hi), arch in AMD_FAMILIES.get(fam, {}).items():
        if "AMD" in fields.get("vendor_id", "") + name and lo <= mod <= hi:
            out += ": " + arch
    if "cache size" in fields:
        out += ", cache %s" % fields["cache size"]
    if "cpu MHz" in fields:
        out += ", %s MHz" % fields["cpu MHz"].split(".")[0]
    return out + ")"


def _oracle():
    """The oracle's single-thread -O2 build (liboracle_cpu.so), used only as the
    timed CPU baseline."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.use_cpu_baseline_build()
    O.set_threads(1)
    return O


def cpu_baseline(seconds=10.0, decode_state=None):
    """The oracle's Q8_0 matvec (the C restatement of the reference's CPU
    arithmetic, built -O2 -ffp-contract=off, one thread) over the same shapes;
    lm_head limited to its first 15,193 rows (a tenth) so one pass stays short.
    Repeats passes until `seconds` of CPU time have elapsed. With the decode
    leg's state, also 16 oracle decode steps after the 512-token prompt."""
    O = _oracle()
    work = []
    for name, N, K, pair in SHAPES:
        rows = 15193 if name == "lm_head" else N
        for i in range(2 if pair else 1):
            raw = uq.synth_quant(uq.KIND_Q8_0, 0xC0FFEE + i * 7 + N, rows, K)
            x = uq.synth_normal(0x5EED0001 + K, K)
            work.append((raw, K, rows, x))
    total_bytes = 0
    passes = 0
    t0 = time.perf_counter()
    while True:
        for raw, K, rows, x in work:
            O.matvec(O.Q8_0, raw, K, rows, x)
            total_bytes += q8_bytes(rows, K)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    out = {"value": round(total_bytes / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": "oracle Q8_0 matvec (int8 activations, exact block sums; gcc -O2 -ffp-contract=off, one "
                     "thread), %d passes over q/o, k/v, gate, up, down and the first 15193 lm_head rows; %.1f s; "
                     "host CPU %s, nproc %d" % (passes, el, cpu_model(), os.cpu_count() or 0)}
    if decode_state is not None:
        out["decode"] = cpu_decode(O, decode_state)
    return out


def cpu_decode(O, st, steps=16):
    """16 greedy steps of the oracle decoder (one thread) on the full
    Qwen2.5-1.5B-shape model at positions 512..527. The oracle's KV cache for
    the 512-token prompt is taken from the GPU prefill (bit-identical to the
    oracle's own prefill in the parity tests; an oracle prefill on one core
    would take tens of minutes). The ids are checked against the GPU's."""
    cfg, tensors, first, gpu_ids, kv = st["cfg"], st["tensors"], st["first"], st["ids"], st["kv"]
    o = O.Model(cfg, {k: v[3] for k, v in tensors.items()})
    for layer, (k, v) in enumerate(kv):
        o.set_kv(layer, k, v)
    tok, ids = first, []
    t0 = time.perf_counter()
    for i in range(steps):
        rc, tok, _ = o.decode(tok, st["prompt"] + i)
        if rc:
            raise RuntimeError("oracle decode rc=%d" % rc)
        ids.append(tok)
    el = time.perf_counter() - t0
    return {"tok_s": round(steps / el, 3), "ms_per_token": round(el * 1e3 / steps, 1), "steps": steps,
            "positions": [st["prompt"], st["prompt"] + steps - 1], "cores": 1,
            "ids_match_gpu": [int(i) for i in ids] == [int(i) for i in gpu_ids[:steps]],
            "sample": "oracle decode (exact-double reductions, int8 activations, fp16 KV) of the 28-layer "
                      "model, %d steps after the 512-token prompt, %.1f s" % (steps, el)}


def decode_bench(prompt_len=512, steps=128, keep=None):
    """Qwen2.5-1.5B-architecture Q8_0 greedy run, bs=1, random-init weights: a
    512-token prompt of seeded uniform ids through the int8-MFMA prefill, then
    `steps` decode steps (one hipGraph launch each, greedy id fed back on the
    device) timed with HIP events. Prefill is timed on the host clock around
    the synchronous call (4 warm-up calls, then the minimum and median of 5). `keep` (a dict) receives what the CPU decode
    baseline needs: the tensors, the prompt's KV cache and the ids."""
    cfg = dict(uq.QWEN25_15B, max_seq=1024)
    t0 = time.perf_counter()
    tensors = uq.synth_qwen2(cfg, 0x5EED0002)
    model = uq.Qwen2Model(cfg, tensors)
    t_load = time.perf_counter() - t0
    prompt = uq.synth_tokens(0x5EED0002, prompt_len, cfg["vocab"])
    # warm-up: after the idle model upload the first prefills run while the
    # clocks ramp (4.95, 4.77, 4.63, 4.53 ms by HIP events on consecutive calls)
    for _ in range(4):
        model.prefill(prompt)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        first = model.prefill(prompt)
        times.append(time.perf_counter() - t0)
    t_prefill = min(times)
    model.decode_run(first, prompt_len, 8)            # warm-up over the same positions
    ids, ms = model.decode_run(first, prompt_len, steps)
    weight_bytes = 28 * 49717248 + 247959552
    kv_bytes = sum(28 * 2 * (prompt_len + i + 1) * 256 * 2 for i in range(steps))
    if keep is not None:                              # decode_run wrote positions 512.., the prompt's KV is intact
        keep.update(cfg=cfg, tensors=tensors, first=int(first), ids=[int(i) for i in ids], prompt=prompt_len,
                    kv=[model.kv(layer, prompt_len) for layer in range(cfg["layers"])])
    model.free()
    return {"tok_s": round(steps / (ms / 1e3), 2), "ms_per_token": round(ms / steps, 4), "prompt": prompt_len,
            "steps": steps, "weight_bytes_per_token": weight_bytes,
            "effective_GBs": round((weight_bytes * steps + kv_bytes) / (ms / 1e3) / 1e9, 1),
            "prefill_tok_s": round(prompt_len / t_prefill, 1), "prefill_ms": round(t_prefill * 1e3, 3),
            "prefill_ms_median": round(sorted(times)[len(times) // 2] * 1e3, 3),
            "model_upload_s": round(t_load, 1), "first_ids": [int(first)] + [int(i) for i in ids[:7]]}


# VALU lane-operations per second of the chip: 256 CUs x 4 SIMDs x 16 lanes
# x 2.4 GHz (packed FP32 not used). The prefill GEMM keeps the reference's
# per-block f32 update, a convert and an fmaf per output and 32-block on the
# VALU (the scale product comes from an f32 outer-product MFMA), so
# 2 x M x N x K/32 lane-operations bound each launch from below.
VALU_LANE_OPS = 256 * 4 * 16 * 2.4e9


def prefill_gemm_bench(tokens=512, reps=20):
    """512-token Q8_0 prefill GEMMs (N x K) 1536x1536, 256x1536, 8960x1536 gate+up
    pair (one fused launch), 1536x8960 on int8 MFMA: TOPS = 2*M*N*K / time,
    against the 5.0 POPS int8 peak and each launch's VALU floor. The model runs
    q|k|v as one N = 2048 launch over the shared input: that launch and the
    model layer's four launches are reported beside the shapes above."""
    out = {}
    tot_ops, tot_ms = 0, 0.0
    layer_ops, layer_ms = 0, 0.0
    shapes = SHAPES[:4] + [("attn_q|k|v", 2048, 1536, False)]
    for name, N, K, pair in shapes:
        w = uq.Weight(uq.KIND_Q8_0, K, N, uq.synth_quant(uq.KIND_Q8_0, 0xABC + N + K, N, K))
        w2 = uq.Weight(uq.KIND_Q8_0, K, N, uq.synth_quant(uq.KIND_Q8_0, 0xABD + N + K, N, K)) if pair else None
        ms = uq.time_prefill_gemm(w, w2, tokens, reps)
        ops = 2 * tokens * N * K * (2 if pair else 1)
        floor_us = 2 * tokens * N * (K // 32) * (2 if pair else 1) / VALU_LANE_OPS * 1e6
        out[name] = {"ms": round(ms, 4), "TOPS": round(ops / (ms / 1e3) / 1e12, 2),
                     "frac_of_int8_peak": round(ops / (ms / 1e3) / 1e12 / 5000.0, 4),
                     "valu_floor_us": round(floor_us, 2), "frac_of_valu_floor": round(floor_us / (ms * 1e3), 3)}
        if name != "attn_q|k|v":
            tot_ops += ops
            tot_ms += ms
        if name != "attn_k/v":
            # one layer of the model: q|k|v, o (the q/o shape), gate+up, down
            layer_ops += ops
            layer_ms += ms
        w.free()
        if w2:
            w2.free()
    out["aggregate_TOPS"] = round(tot_ops / (tot_ms / 1e3) / 1e12, 2)
    out["model_layer_TOPS"] = round(layer_ops / (layer_ms / 1e3) / 1e12, 2)
    out["model_layer_ms"] = round(layer_ms, 4)
    out["int8_mfma_peak_TOPS"] = 5000.0
    return out


def prefill_attention_bench(tokens=512, heads=12, kv_heads=2, head_dim=128, reps=50):
    """The 512-token prefill's causal attention alone (Qwen2.5-1.5B heads: 12 query,
    2 KV, head_dim 128; int8 output planes for the o GEMM as in the model), HIP
    events over `reps` launches. Causal flops = 2 contractions x 2 x head_dim x
    (1 + 2 + ... + tokens) per head; issued = what the 16-query x 16-key tiles
    of v_mfma_f64_16x16x4_f64 execute (q.k over whole 16-key tiles, P.V over
    whole 4-key steps)."""
    ms = uq.time_prefill_attention(tokens, heads, kv_heads, head_dim, True, reps)
    causal = heads * 2 * 2 * head_dim * tokens * (tokens + 1) // 2
    issued = 0
    for t0 in range(0, tokens, 16):
        kend = t0 + min(16, tokens - t0)
        issued += 16 * 16 * 2 * head_dim * (((kend + 15) // 16) + ((kend + 3) // 4 * 4) / 16)
    issued *= heads
    return {"us": round(ms * 1e3, 2), "causal_TFLOPs": round(causal / (ms / 1e3) / 1e12, 2),
            "issued_TFLOPs": round(issued / (ms / 1e3) / 1e12, 2), "fp64_mfma_peak_TFLOPs": 78.6,
            "issued_frac": round(issued / (ms / 1e3) / 1e12 / 78.6, 4),
            "shape": "%d tokens, %d/%d heads, head_dim %d" % (tokens, heads, kv_heads, head_dim)}


def mfma_probe():
    """Matrix-core rates on this GPU: 16 waves per CU (kinds 0-2), and one wave per
    SIMD with and without the VALU work the prefill kernels put beside their
    MFMAs (kinds 3-6): fp64 MFMAs with an fp16 -> double operand conversion each,
    int8 MFMAs beside the per-block f32 rescale."""
    r = {"int8_TOPS": round(uq.probe_mfma(0), 1), "int8_32x32x32_TOPS": round(uq.probe_mfma(9), 1),
         "int8_16x16x64_TOPS": round(uq.probe_mfma(10), 1), "fp16_TFLOPS": round(uq.probe_mfma(1), 1),
         "fp64_TFLOPS": round(uq.probe_mfma(2), 1)}
    one = {k: uq.probe_mfma(kind) for k, kind in (("fp64", 3), ("fp64_and_conv", 4), ("conv_only", 5),
                                                  ("int8", 6), ("int8_and_rescale", 7), ("rescale_only", 8))}
    # iteration time ~ 1/rate: additive work gives 1/both = 1/mfma + 1/valu,
    # full overlap gives 1/both = max(1/mfma, 1/valu)
    overlap = lambda m, b, v: round((1 / m + 1 / v - 1 / b) / min(1 / m, 1 / v), 3)
    r["one_wave_per_simd"] = {k: round(v, 1) for k, v in one.items()}
    r["one_wave_per_simd"]["fp64_overlap"] = overlap(one["fp64"], one["fp64_and_conv"], one["conv_only"])
    r["one_wave_per_simd"]["int8_overlap"] = overlap(one["int8"], one["int8_and_rescale"], one["rescale_only"])
    r["note"] = ("independent chains of v_mfma_i32_16x16x32_i8 (int8_TOPS) / v_mfma_i32_32x32x32_i8 / "
                 "v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_f16 / v_mfma_f64_16x16x4_f64 "
                 "on register operands, 16 waves per CU, same GPU; one_wave_per_simd: 16 MFMAs per iteration on "
                 "4 chains and/or the VALU work beside them (fp64: 16 fp16->double operand conversions; int8: "
                 "convert, scale product, fma of 16 f32 accumulators), rates of the same MFMA count; overlap: "
                 "share of the shorter part hidden under the longer (0 additive, 1 fully overlapped)")
    return r


def kquant_sweep(kind, copies=3, reps=30):
    """The same bs=1 sweep with K-quant weights: Q4_K (144 B per 256 values)
    or Q3_K (110 B per 256 values); lm_head alone timed over back-to-back
    launches."""
    bpsb = {uq.KIND_Q4_K: 144, uq.KIND_Q3_K: 110}[kind]
    weights, pairs, names = [], [], []
    for c in range(copies):
        for name, N, K, pair in SHAPES:
            for i in range(2 if pair else 1):
                raw = uq.synth_quant(kind, 0x5EED0011 + kind * 256 + c * 16 + i * 4 + N, N, K)
                weights.append(uq.Weight(kind, K, N, raw))
                pairs.append(1 if (pair and i == 0) else 0)
                names.append(name)
    kb = lambda N, K: N * (K // 256) * bpsb + K + (K // 32) * 4 + 4 * N
    step_bytes = sum(kb(N, K) * 2 - (K + K // 32 * 4) - 4 * N if pair else kb(N, K) for _, N, K, pair in SHAPES)
    total_ms, _ = uq.time_matvecs(weights, pairs, 8960, reps, 3, -1)
    lm_ws = [w for w, n in zip(weights, names) if n == "lm_head"]
    lm_total, _ = uq.time_matvecs(lm_ws, [0] * len(lm_ws), 1536, reps, 3, -1)
    lm_ms = lm_total / (reps * len(lm_ws))
    for w in weights:
        w.free()
    return {"GBs": round(step_bytes * reps * copies / (total_ms / 1e3) / 1e9, 1), "bytes_per_step": step_bytes,
            "lm_head_GBs": round(kb(151936, 1536) / (lm_ms / 1e3) / 1e9, 1),
            "lm_head_frac": round(kb(151936, 1536) / (lm_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}


def q4k_sweep():
    return kquant_sweep(uq.KIND_Q4_K)


def q3k_sweep():
    return kquant_sweep(uq.KIND_Q3_K)


def moe_bench(steps=64):
    """MoE decode layer: 128 Q3_K experts (dim 2048, ff 768), top-8 softmax
    routing from N(0,1) logits, one shared Q8_0 expert; 64 seeded steps back to
    back. Bytes per step: 8 x 3 Q3_K expert matrices + 3 shared Q8_0 matrices."""
    cfg = uq.MOE_CONFIG
    ex, sh, gi = uq.synth_moe(cfg, 0x5EED0004)
    layer = uq.MoeLayer(cfg, ex, sh, gi)
    xs = np.stack([uq.synth_normal(0x5EED0004 + 1000 * s, cfg["dim"]) for s in range(steps)])
    lg = np.stack([uq.synth_normal(0x5EED0004 + 1000 * s + 1, cfg["experts"]) for s in range(steps)])
    layer.run(xs[:4], lg[:4])
    _, ms = layer.run(xs, lg)
    layer.free()
    step_bytes = 8 * 2027520 + 5013504
    return {"GBs": round(step_bytes * steps / (ms / 1e3) / 1e9, 1), "us_per_step": round(ms * 1e3 / steps, 2),
            "steps": steps, "bytes_per_step": step_bytes}


LINEAR_NAMES = {uq.KIND_F32: "F32", uq.KIND_BF16: "BF16", uq.KIND_Q8_0: "Q8_0", uq.KIND_Q6_K: "Q6_K",
                uq.KIND_IQ3_XXS: "IQ3_XXS", uq.KIND_IQ4_NL: "IQ4_NL", uq.KIND_IQ4_XS: "IQ4_XS"}


def linear_sweep(n=2560, copies=3, reps=20):
    """fp32-activation reader (the frontier backend's matvec): per kind one
    m x 2560 weight of about 128 MB, 3 rotating copies (more than the 256 MB
    MALL), one launch per copy in turn. Bytes per launch: the GGUF weight
    bytes + 4n (x) + 4m (y)."""
    out = {}
    for kind in uq.LINEAR_KINDS:
        rb = uq.row_bytes(kind, n)
        m = min(160000, (128 << 20) // rb)
        ws = [uq.Weight(kind, n, m, uq.synth_quant(kind, 0x5EED0020 + 16 * kind + c, m, n)) for c in range(copies)]
        ms = uq.time_linear(ws, reps, 2)
        for w in ws:
            w.free()
        nbytes = m * rb + 4 * n + 4 * m
        gbs = nbytes * copies * reps / (ms / 1e3) / 1e9
        out[LINEAR_NAMES[kind]] = {"rows": m, "bytes_per_launch": nbytes, "us_per_launch": round(ms * 1e3 / (copies * reps), 2),
                                   "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def launch_cost(reps=200):
    """One Q8_0 matvec launch's mean duration between HIP events after
    different predecessors (the sweep's small q/o and k/v launches)."""
    mk = lambda n, k, seed: uq.Weight(uq.KIND_Q8_0, k, n, uq.synth_quant(uq.KIND_Q8_0, seed, n, k))
    kv = [mk(256, 1536, 0x5EED0031 + i) for i in range(3)]
    qo = mk(1536, 1536, 0x5EED0034)
    lm = mk(151936, 1536, 0x5EED0035)
    down = mk(1536, 8960, 0x5EED0036)
    cases = [("k/v alone", [kv[0]], 0, reps), ("k/v after k/v (three copies)", kv, 1, reps),
             ("q/o alone", [qo], 0, reps), ("k/v after q/o", [qo, kv[0]], 1, reps),
             ("k/v after lm_head", [lm, kv[0]], 1, reps // 3), ("q/o after lm_head", [lm, qo], 1, reps // 3),
             ("k/v after down", [down, kv[0]], 1, reps), ("lm_head alone", [lm], 0, reps // 3)]
    out = {}
    for name, ws, probe, r in cases:
        tot, pm = uq.time_matvecs(ws, [0] * len(ws), 151936, r, 10, probe)
        out[name] = {"probed_us": round(pm * 1000, 2), "round_us": round(tot * 1000 / r, 2)}
    out["note"] = "mean of the probed launch between HIP events (the event records add their own time)"
    return out


def frontier_moe_bench(tokens=32, reps=3, experts=256, top_k=10, dim=2560, ff=640):
    """Device work of the frontier MoE block (Forward::ffn) per token: the F32
    router linear, then the 23-job table (10 routed experts' IQ3_XXS gate and
    up, the shared Q8_0 gate and up, the F32 shared scale) and the 11-job
    table (IQ4_NL routed down, Q8_0 shared down), one launch each. Experts are
    drawn per token (seeded) from a bank of `experts` (about 557 MB for 256,
    more than the MALL). The host arithmetic between the tables is not timed."""
    import ctypes
    rng = np.random.default_rng(0x5EED0005)
    mk = lambda kind, n, m, seed: uq.Weight(kind, n, m, uq.synth_quant(kind, seed, m, n))
    router = mk(uq.KIND_F32, dim, experts, 1)
    sscale = mk(uq.KIND_F32, dim, 1, 2)
    sgate, sup = mk(uq.KIND_Q8_0, dim, ff, 3), mk(uq.KIND_Q8_0, dim, ff, 4)
    sdown = mk(uq.KIND_Q8_0, ff, dim, 5)
    gate = [mk(uq.KIND_IQ3_XXS, dim, ff, 100 + e) for e in range(experts)]
    up = [mk(uq.KIND_IQ3_XXS, dim, ff, 10000 + e) for e in range(experts)]
    down = [mk(uq.KIND_IQ4_NL, ff, dim, 20000 + e) for e in range(experts)]
    L = uq.lib()
    nbuf = dim + experts + 23 * ff + 11 * ff + 11 * dim
    buf = ctypes.c_void_p()
    uq._check(L.uq_dev_alloc(4 * nbuf, ctypes.byref(buf)))
    uq._check(L.uq_memcpy_h2d(buf, np.ascontiguousarray(rng.normal(0, 1, nbuf).astype(np.float32)).ctypes.data,
                              4 * nbuf))
    at = lambda off: buf.value + 4 * off
    x, sc = at(0), at(dim)
    proj = [at(dim + experts + i * ff) for i in range(23)]
    mid = [at(dim + experts + (23 + i) * ff) for i in range(11)]
    outs = [at(dim + experts + 34 * ff + i * dim) for i in range(11)]
    jobs, sizes = [], []
    for t in range(tokens):
        ids = rng.choice(experts, top_k, replace=False)
        jobs.append(uq.LinearJob(router.handle, x, sc))
        sizes.append(1)
        a = []
        for e in ids:
            a += [uq.LinearJob(gate[e].handle, x, proj[len(a)]), uq.LinearJob(up[e].handle, x, proj[len(a) + 1])]
        a += [uq.LinearJob(sgate.handle, x, proj[20]), uq.LinearJob(sup.handle, x, proj[21]),
              uq.LinearJob(sscale.handle, x, proj[22])]
        jobs += a
        sizes.append(len(a))
        b = [uq.LinearJob(down[e].handle, mid[i], outs[i]) for i, e in enumerate(ids)]
        b.append(uq.LinearJob(sdown.handle, mid[10], outs[10]))
        jobs += b
        sizes.append(len(b))
    jt = (uq.LinearJob * len(jobs))(*jobs)
    st = (ctypes.c_int * len(sizes))(*sizes)
    ms = ctypes.c_double()
    uq._check(L.uq_time_linear_tables(jt, st, len(sizes), reps, ctypes.byref(ms)))
    L.uq_dev_free(buf)
    for w in [router, sscale, sgate, sup, sdown] + gate + up + down:
        w.free()
    us = ms.value * 1e3 / (reps * tokens)
    step_bytes = (experts * dim * 4 + top_k * (2 * ff * 980 + dim * (ff // 32) * 18) + 3 * ff * (dim // 32) * 34
                  + dim * 4)
    return {"us_per_token_layer": round(us, 2), "GBs": round(step_bytes / (us * 1e-6) / 1e9, 1),
            "bytes_per_token_layer": step_bytes, "launches_per_token_layer": 3, "tokens": tokens, "experts": experts}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=3, help="rotating weight copies (> 256 MB MALL in total)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the full-model decode leg")
    ap.add_argument("--leg", choices=["decode", "prefill", "attention", "probes", "q4k", "q3k", "moe", "linear",
                                      "frontier_moe", "launches"],
                    help="run only this secondary leg and print its JSON (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU; --gpus %d is not supported "
              "(the path's multi-GPU sharding is design-only)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    uq.init(0)
    if args.leg:
        leg = {"decode": decode_bench, "prefill": prefill_gemm_bench, "attention": prefill_attention_bench,
               "probes": mfma_probe,
               "q4k": q4k_sweep, "q3k": q3k_sweep,
               "moe": moe_bench, "linear": linear_sweep, "frontier_moe": frontier_moe_bench,
               "launches": launch_cost}[args.leg]
        print(json.dumps({args.leg: leg()}), flush=True)
        return
    weights, pairs, shape_of = [], [], []
    for c in range(args.copies):
        for name, N, K, pair in SHAPES:
            for i in range(2 if pair else 1):
                raw = uq.synth_quant(uq.KIND_Q8_0, (0x5EED0001 << 8) + c * 16 + i * 4 + N, N, K)
                weights.append(uq.Weight(uq.KIND_Q8_0, K, N, raw))
                pairs.append(1 if (pair and i == 0) else 0)
                shape_of.append((name, N, K, pair))
    per_copy = len(weights) // args.copies
    # a fused pair reads two weight matrices and one activation, writes one output
    step_bytes = sum(q8_bytes(N, K) * 2 - (K + K // 32 * 4) - 4 * N if pair else q8_bytes(N, K)
                     for _, N, K, pair in SHAPES)
    steps, warmup = args.steps, args.warmup
    # step j runs weight copy j % copies: warmup steps 0..W-1 untimed, then
    # exactly K timed steps W..W+K-1 between one HIP event pair
    def step_list(first, count, order=None):
        ws, ps = [], []
        for j in range(first, first + count):
            chunk = range((j % args.copies) * per_copy, (j % args.copies + 1) * per_copy)
            for i in (sorted(chunk, key=order) if order else chunk):
                ws.append(weights[i])
                ps.append(pairs[i])
        return ws, ps

    def timed(fn, order=None):
        if warmup:
            fn(*step_list(0, warmup, order))
        return fn(*step_list(warmup, steps, order))

    total_ms = timed(lambda ws, ps: uq.time_matvecs(ws, ps, 8960, 1, 0, -1)[0])
    value = step_bytes * steps / (total_ms / 1e3) / 1e9
    # the same matvecs with each copy's weights of one input length in one
    # job-table launch (q/o, k/v, gate+up pair, lm_head at K=1536; down at
    # K=8960), the graph_linear table form, reported beside `value`
    by_k = lambda i: (shape_of[i][2], i)
    tables_ms = timed(lambda ws, ps: uq.time_matvec_tables(ws, ps, 8960, 1, 0), order=by_k)
    tables_gbs = step_bytes * steps / (tables_ms / 1e3) / 1e9
    # dominant kernel alone: lm_head launches back to back over the copies,
    # one event pair around all of them -> mean launch duration
    lm_ws = [w for w, sh in zip(weights, shape_of) if sh[0] == "lm_head"]
    lm_rounds = max(1, steps // args.copies)
    lm_total, _ = uq.time_matvecs(lm_ws, [0] * len(lm_ws), 1536, lm_rounds, 1, -1)
    lm_ms = lm_total / (lm_rounds * len(lm_ws))
    lm_bytes = q8_bytes(151936, 1536)
    lm_gbs = lm_bytes / (lm_ms / 1e3) / 1e9

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(total_ms / steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q8_0 matvec sweep bs=1, Qwen2.5-1.5B shapes (NxK) 1536x1536, 256x1536, "
                               "2x8960x1536 fused gate+up, 1536x8960, 151936x1536; %d rotating weight copies"
                               % args.copies,
                   "bytes_per_step": step_bytes, "seed": 0x5EED0001, "fraction_of_hbm_peak":
                       round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(lm_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": LM_HEAD_TRAFFIC_BYTES,
                     "kernel": "Q8_0 matvec, lm_head 151936x1536 (%d B per launch), mean of %d back-to-back "
                               "launches %.4f ms" % (lm_bytes, lm_rounds * len(lm_ws), lm_ms)},
    }
    result["sweep_job_tables"] = {
        "GBs": round(tables_gbs, 2), "frac": round(tables_gbs / HBM_PEAK_GBS, 4),
        "ms_per_step": round(tables_ms / steps, 5),
        "note": "same weights and bytes; per step two launches (the four K=1536 matvecs as one job table, "
                "down alone) instead of five"}
    read_gbs, copy_gbs = uq.probe_bandwidth(1 << 30, 10)
    result["hbm_probe"] = {"stream_read_GBs": round(read_gbs, 1), "copy_GBs": round(copy_gbs, 1),
                           "note": "streaming read of 1 GiB (one 28 KB chunk of non-temporal 16-byte loads per "
                                   "workgroup) and plain int4 copy, same GPU"}
    result["mfma_probe"] = mfma_probe()
    for w in weights:
        w.free()
    decode_state = {} if not args.no_cpu else None
    if not args.no_decode:
        result["decode"] = decode_bench(keep=decode_state)
        result["prefill_gemm"] = prefill_gemm_bench()
        pg = result["prefill_gemm"]
        pg["frac_of_int8_peak"] = round(pg["aggregate_TOPS"] / pg["int8_mfma_peak_TOPS"], 4)
        pg["measured_32x32x32_TOPS"] = result["mfma_probe"]["int8_32x32x32_TOPS"]
        result["prefill_attention"] = prefill_attention_bench()
        result["q4k_sweep"] = q4k_sweep()
        result["q3k_sweep"] = q3k_sweep()
        result["moe"] = moe_bench()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(decode_state=decode_state or None)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
