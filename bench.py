#!/usr/bin/env python3
"""Benchmark of the akasha-core inference hot path on one MI355X.

Headline metric (config 4): akasha-hall 1.0 fp32 greedy
decode at batch 32 -- every sequence prefilled with 448 random tokens
(seed 4), then decode steps at positions 448..511 so the KV cache reaches
512 tokens.  A "step" is one decode step of all 32 sequences (embedding ->
12 layers -> lm_head -> argmax, graph-replayed, tokens fed back on the
device).  ``value`` = 32 * steps / time (tok/s), inputs resident in HBM.
The timed steps are always whole windows of 64 at positions 448..511 (KV
449..512): ``--steps K`` times ceil(K / 64) windows, the cache truncated
back to 448 between them, and the line reports the steps actually timed.

Also reported: the roofline of the dominant decode kernel (single-query
attention over the cache, its launches cycled over the layers and timed
with HIP events on the session's stream), the whole-step HBM
roofline, per-kernel times, config-3 prefill (16 x 512) throughput against
the fp32 MFMA peak, and the CPU baseline: the oracle's decode step (a C
restatement of the reference CPU backend) on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__ as entry  # noqa: E402

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2516.6  # dense


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_attn_b32_ctx512_pmc.md"
TRAFFIC_SOURCE = ("not measured in this run: rocprofv3 FETCH_SIZE + WRITE_SIZE passes over the "
                  "same kernel, scaled by a copy kernel, committed in "
                  "profiles/decode_attn_b32_ctx512_pmc.md (regenerated with each change to "
                  "k_dec_attn)")


def measured_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (counters cannot be read from
    inside this process); None if the summary is absent."""
    try:
        for line in Path(path).read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def decode_step_bytes(cfg, B, T):
    """Algorithmic bytes of one decode step whose attention reads T rows:
    weights once, KV rows read, KV append, embedding rows, logits written."""
    d, L, V = cfg.dim, cfg.num_layers, cfg.vocab_size
    weights = 4 * (sum(int(np.prod(s)) for s in cfg.param_shapes()) - V * d)
    kv_read = 2 * L * B * T * d * 4
    kv_append = 2 * L * B * d * 4
    return weights + kv_read + kv_append + B * d * 4 + B * V * 4


def prefill_flop_parts(cfg, B, S, lm_rows=None):
    """(layer GEMM, attention, lm_head) flops of a B x S prefill; lm_head on
    `lm_rows` rows (default: the last row of every sequence)."""
    d, F, L, H, hd, V = cfg.dim, cfg.ffn_hidden, cfg.num_layers, cfg.num_heads, cfg.head_dim, cfg.vocab_size
    gemm = 2 * B * S * L * (d * 3 * d + d * d + d * F + F * d)
    attn = 2 * hd * S * (S + 1) * B * H * L
    lm = 2 * (B if lm_rows is None else lm_rows) * d * V
    return gemm, attn, lm


def prefill_rates(ms, gemm, attn, lm, h3_flop, x6_flop):
    """Rates of a prefill that took `ms`.

    - `tflops`: useful fp32 work per second (2 x multiply-adds of the GEMMs,
      the causal attention pairs and the lm_head rows).
    - `fp32_equiv_over_fp32_peak`: that rate over the fp32 MFMA peak.  It is
      not a fraction of any ceiling when the work runs on 16-bit MFMAs (it
      can exceed 1): it says how the kernels compare with fp32 arithmetic.
    - `roofline`: the MFMA work the kernels execute against the peak of the
      instructions that execute it.  The split-fp16 kernels (`h3_flop` of the
      useful flops) run three fp16 products per fp32 multiply-add, the
      split-bfloat16 ones (`x6_flop`) six bf16 products, both on 16-bit MFMAs
      (2516.6 TFLOP/s dense); the rest runs on fp32 MFMAs (157.3).  `frac`
      = the time those pipes need at their peaks / the elapsed time."""
    t = ms / 1e3
    useful = gemm + attn + lm
    exec16 = 3 * h3_flop + 6 * x6_flop
    exec32 = useful - h3_flop - x6_flop
    busy = exec16 / (BF16_MFMA_PEAK_TFLOPS * 1e12) + exec32 / (FP32_MFMA_PEAK_TFLOPS * 1e12)
    if exec16:
        instr = ("v_mfma_f32_32x32x16_f16, 3 products per fp32 multiply-add" if h3_flop
                 else "v_mfma_f32_32x32x16_bf16, 6 products per fp32 multiply-add")
        roof = {"bound": "mfma", "instr": instr, "achieved": round(exec16 / t / 1e12, 2),
                "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(busy / t, 4)}
    else:
        roof = {"bound": "mfma", "instr": "v_mfma_f32_32x32x2_f32",
                "achieved": round(exec32 / t / 1e12, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(busy / t, 4)}
    return {"tflops": round(useful / t / 1e12, 2),
            "fp32_equiv_over_fp32_peak": round(useful / t / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
            "roofline": roof}


def scaled_decode(hip, be, model, cfg, T, steps):
    """Config 5 decode legs: 64 sequences in one session (two 32-row MFMA
    tiles sharing every weight read), `steps` steps ending at KV length T,
    with the f32 KV cache and then the optional bfloat16 one.  The weights
    are bf16-valued and read as bfloat16 tiles, so their algorithmic bytes
    are 2 per parameter, read once per step."""
    d, L, V = cfg.dim, cfg.num_layers, cfg.vocab_size
    B = 64
    weights = 2 * (sum(int(np.prod(x)) for x in cfg.param_shapes()) - V * d)
    kv = sum(2 * L * B * (T - steps + i + 1) * d * 4 for i in range(steps))
    s = hip.Session(model, T, B)
    out = {"decode_workload": f"{B} sequences in one session, {steps} steps to KV length "
                              f"{T}, KV rows before them filled with N(0, 1) values "
                              f"(akh_session_fill_cache_synthetic, seed 6)",
           "decode_launches_per_step": s.decode_launches()}
    for kv16 in (False, True):
        if kv16:
            s.set_len(0)
            s.set_kv_bf16(True)
        s.fill_cache_synthetic(T - steps, 6)
        s.decode_greedy(1, want_tokens=False)  # capture + warm
        s.set_len(T - steps)
        be.synchronize()
        be.timer_start()
        s.decode_greedy(steps, want_tokens=False)
        ms = be.timer_stop()
        step_bytes = (weights * steps + (kv / 2 if kv16 else kv)) / steps
        key = "decode_kv16" if kv16 else "decode"
        out.update({f"{key}_ms_per_step": round(ms / steps, 3),
                    f"{key}_tok_s": round(B * steps / (ms / 1e3), 1),
                    f"{key}_hbm_frac": round(step_bytes / (ms / steps / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                    f"{key}_bytes_per_step": int(step_bytes)})
    s.close()
    return out


DECODE_KERNELS = ["decode_attn", "qkv_proj", "out_proj", "ffn_up", "ffn_down",
                  "lm_head_argmax", "resid_norm"]


def decode_kernel_legs(sess, cfg, B, T, reps, wbytes=4, kvbytes=4):
    """Each decode kernel alone: `reps` back-to-back launches cycled over the
    layers (each reads its layer's weights and KV rows as in a step), at KV
    length T, timed by two events around them (gaps included).  Returns
    ({name: ms, algorithmic bytes, GB/s}, attention ms per dispatch from
    events the dispatches carry themselves).  Algorithmic bytes per launch:
    weights once (`wbytes` per parameter), activations in and out once."""
    kms = {n: sess.time_decode_kernel(i, reps) for i, n in enumerate(DECODE_KERNELS)}
    attn_dispatch_ms = sess.time_decode_attn(reps)
    d, V, F = cfg.dim, cfg.vocab_size, cfg.ffn_hidden
    kbytes = {
        "decode_attn": 2 * B * T * d * kvbytes + 2 * B * d * kvbytes,
        "qkv_proj": d * 3 * d * wbytes + B * 4 * d * 4,
        "out_proj": d * d * wbytes + 2 * B * d * 4,
        "ffn_up": d * F * wbytes + B * (d + F) * 4,
        "ffn_down": F * d * wbytes + B * (F + d) * 4,
        "lm_head_argmax": d * V * wbytes + B * d * 4 + B * V * 4,
        "resid_norm": 4 * B * d * 4 + d * 4,
    }
    kernels = {n: {"ms": round(kms[n], 5), "bytes": kbytes[n],
                   "GB/s": round(kbytes[n] / (kms[n] / 1e3) / 1e9, 1)} for n in DECODE_KERNELS}
    return kernels, attn_dispatch_ms


def kernel_legs_only(pkg, hip, be, model, cfg, reps, scaled):
    """The per-kernel decode legs without any graph replay (for counter
    runs): config 4 at T = 481 after a 32 x 448 prefill with the KV length
    then set to 480, and with `scaled` config 5's 64-row session at
    T = 2048 over KV rows filled with N(0, 1) values."""
    B, P, CTX = 32, 448, 512
    sess = hip.Session(model, CTX, B)
    prompt = pkg.synthetic_tokens(B * P, cfg.vocab_size, seed=4).reshape(B, P)
    log("bench: prefill 32 x 448")
    sess.prefill(prompt, want_logits=False)
    sess.set_len(480)
    log(f"bench: config 4 decode kernels, {reps} launches each")
    k4, a4 = decode_kernel_legs(sess, cfg, B, 481, reps)
    # The same legs with the fused norm (akh_session_set_fused_norm): out_proj
    # and ffn_down add their sums to the residual themselves, qkv_proj and
    # ffn_up scale their A operand by the RMSNorm, and the norm kernel that
    # remains is the final norm before the lm_head.
    log(f"bench: config 4 decode kernels with the fused norm, {reps} launches each")
    sess.set_fused_norm(True)
    k4f, _ = decode_kernel_legs(sess, cfg, B, 481, reps)
    sess.set_fused_norm(False)
    sess.close()
    out = {"config4": {"T": 481, "kernels": k4, "attn_dispatch_ms": round(a4, 5)},
           "config4_fused_norm": {"T": 481, "kernels": k4f}}
    if scaled:
        c5 = pkg.ModelConfig.scaled()
        log("bench: scaled config weights (seed 5, bf16 values)")
        w5 = pkg.synthetic_weights(c5, seed=5, bf16=True)
        m5 = hip.Model(be, c5)
        m5.upload(w5)
        del w5
        s5 = hip.Session(m5, 2048, 64)
        s5.fill_cache_synthetic(2047, 6)
        log(f"bench: config 5 decode kernels, {reps} launches each")
        k5, a5 = decode_kernel_legs(s5, c5, 64, 2048, reps, wbytes=2)
        s5.close()
        m5.close()
        out["config5"] = {"T": 2048, "kernels": k5, "attn_dispatch_ms": round(a5, 5)}
    return out


def scaled_measurement(pkg, hip, be, w, steps=8, with_prefill=True, with_decode=True):
    """Config 5: the scaled architecture (dim 2048, 24 layers, 16 x 128, FFN
    8192, vocab 50257) with bf16-valued weights `w` (seed 5).  Decode: 64
    sequences (one session) for `steps` steps ending at KV length
    2048, over KV rows filled with N(0, 1) values.  Prefill: 8 x 2048
    (seed 7)."""
    cfg = pkg.ModelConfig.scaled()
    model = hip.Model(be, cfg)
    model.upload(w)
    T, V = 2048, cfg.vocab_size
    out = {"workload": "config 5: scaled architecture, bf16-valued weights (seed 5)"}
    if with_decode:
        out.update(scaled_decode(hip, be, model, cfg, T, steps))
    if with_prefill:
        Bp, Sp = 8, 2048
        ps = hip.Session(model, Sp, Bp)
        toks = pkg.synthetic_tokens(Bp * Sp, V, seed=7).reshape(Bp, Sp)
        log("bench: scaled config prefill 8 x 2048")
        ps.prefill(toks, want_logits=False)
        ps.reset()
        be.synchronize()
        be.timer_start()
        ps.prefill(toks, want_logits=False)
        pms = be.timer_stop()
        g, a, lm = prefill_flop_parts(cfg, Bp, Sp)
        fl = g + a + lm
        r = prefill_rates(pms, g, a, lm, g + a, 0)
        out.update({"prefill_kernels": "split-fp16 GEMMs and flash (two fp16 terms, three "
                                       "products; fp32-accurate, default)",
                    "prefill_ms": round(pms, 2), "prefill_tok_s": round(Bp * Sp / (pms / 1e3), 1),
                    "prefill_tflops": r["tflops"],
                    "prefill_fp32_equiv_over_fp32_peak": r["fp32_equiv_over_fp32_peak"],
                    "prefill_roofline": r["roofline"]})
        # The same prefill with the layer GEMMs and flash on the fp32 MFMAs.
        log("bench: scaled config prefill 8 x 2048, fp32 MFMAs")
        split = model.prefill_split()
        model.set_prefill_split(hip.Model.SPLIT_NONE)
        ps.reset()
        ps.prefill(toks, want_logits=False)
        ps.reset()
        be.synchronize()
        be.timer_start()
        ps.prefill(toks, want_logits=False)
        fms = be.timer_stop()
        model.set_prefill_split(split)
        out.update({"prefill_fp32_mfma_ms": round(fms, 2),
                    "prefill_fp32_mfma_tok_s": round(Bp * Sp / (fms / 1e3), 1),
                    "prefill_fp32_mfma_roofline": prefill_rates(fms, g, a, lm, 0, 0)["roofline"]})
        # The optional bf16-MFMA prefill (logits within 2e-2 of f32).
        log("bench: scaled config prefill 8 x 2048, bf16 MFMA")
        model.set_prefill_bf16(True)
        ps.reset()
        ps.prefill(toks, want_logits=False)
        ps.reset()
        be.synchronize()
        be.timer_start()
        ps.prefill(toks, want_logits=False)
        bms = be.timer_stop()
        model.set_prefill_bf16(False)
        out.update({"prefill_bf16_ms": round(bms, 2),
                    "prefill_bf16_tok_s": round(Bp * Sp / (bms / 1e3), 1),
                    "prefill_bf16_tflops": round(fl / (bms / 1e3) / 1e12, 2),
                    "prefill_bf16_roofline": {
                        "bound": "mfma",
                        "instr": "v_mfma_f32_32x32x16_bf16; useful flops counted once (ffn_up and "
                                 "ffn_down run two products, hi + lo of their fp32 input)",
                        "achieved": round(fl / (bms / 1e3) / 1e12, 2),
                        "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(fl / (bms / 1e3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4)}})
        ps.close()
    model.close()
    return out


def prefill_measurement(pkg, hip, be, model, cfg, CTX, reps=3):
    """Config 3 (16 x 512 prefill, seed 3) on the default split-fp16 kernels,
    on the split-bf16 ones and on the fp32 MFMAs, then the trainer forward on
    the same rows."""
    Bp, Sp = 16, 512
    ps = hip.Session(model, CTX, Bp)
    ptoks = pkg.synthetic_tokens(Bp * Sp, cfg.vocab_size, seed=3).reshape(Bp, Sp)
    ps.prefill(ptoks, want_logits=False)  # warm
    times = []
    for _ in range(reps):
        ps.reset()
        be.synchronize()
        be.timer_start()
        ps.prefill(ptoks, want_logits=False)
        times.append(be.timer_stop())
    pms = min(times)
    g, a, lm = prefill_flop_parts(cfg, Bp, Sp)
    fl = g + a + lm
    prefill = {"workload": "config 3: hall-1.0 fp32 prefill 16 x 512 (seed 3), last-row logits",
               "kernels": "split-fp16 GEMMs and flash (fp32 operands as two fp16 terms, three "
                          "products); fp32-accurate, the default",
               "ms": round(pms, 3), "tok_s": round(Bp * Sp / (pms / 1e3), 1),
               **prefill_rates(pms, g, a, lm, g + a, 0), "flop": fl}
    split = model.prefill_split()

    def timed(kind):
        model.set_prefill_split(kind)
        ps.reset()
        ps.prefill(ptoks, want_logits=False)  # warm
        ts = []
        for _ in range(reps):
            ps.reset()
            be.synchronize()
            be.timer_start()
            ps.prefill(ptoks, want_logits=False)
            ts.append(be.timer_stop())
        return min(ts)

    # The same prefill with the GEMMs and flash split into three bfloat16 terms.
    x6 = timed(hip.Model.SPLIT_X6)
    prefill["split_bf16_x6"] = {"ms": round(x6, 3), "tok_s": round(Bp * Sp / (x6 / 1e3), 1),
                                **prefill_rates(x6, g, a, lm, 0, g + a)}
    # The same prefill with the layer GEMMs and flash on the fp32 MFMAs.
    p32 = timed(hip.Model.SPLIT_NONE)
    model.set_prefill_split(split)
    prefill["fp32_mfma"] = {"ms": round(p32, 3), "tok_s": round(Bp * Sp / (p32 / 1e3), 1),
                            "tflops": round(fl / (p32 / 1e3) / 1e12, 2),
                            **{k: v for k, v in prefill_rates(p32, g, a, lm, 0, 0).items()
                               if k == "roofline"}}
    ps.close()
    # Trainer::forward + CrossEntropy on the same 16 x 512 rows: the
    # lm_head runs on every row (+2 rows d V flop) and the loss follows.
    fw = hip.Forward(model, Bp, Sp)
    targets = np.roll(ptoks, -1, axis=1)
    fw.loss(ptoks, targets)  # warm
    ftimes = []
    for _ in range(reps):
        be.synchronize()
        be.timer_start()
        mean_loss, _ = fw.loss(ptoks, targets)
        ftimes.append(be.timer_stop())
    fms = min(ftimes)
    g, a, flm = prefill_flop_parts(cfg, Bp, Sp, lm_rows=Bp * Sp)
    ffl = g + a + flm
    prefill["train_forward"] = {
        "workload": "Trainer::forward + CrossEntropy, 16 x 512 rows (seed 3), all-rows lm_head",
        "ms": round(fms, 3), "tok_s": round(Bp * Sp / (fms / 1e3), 1),
        **prefill_rates(fms, g, a, flm, g + a + flm, 0),
        "mean_loss": round(mean_loss, 4), "flop": ffl}
    fw.close()
    return prefill


def config2_measurement(hip, be, reps=10):
    """Config 2: the flash-attention op, 8 sequences x 12 heads x 512 x 64,
    N(0,1) from seed 2, scale 1/8.  As the reference issues it: one
    FLASH_ATTENTION node per sequence at row_offset b * 512
    (layers.rs:410-421; each node runs the key-split kernel), and the same
    nodes as one launch (akh_flash_attention_batched).  Both run split-fp16
    tiles (three fp16 products per fp32 multiply-add); a tile with an operand
    beyond fp16's range recomputes itself on split-bfloat16 products (none
    does on these inputs)."""
    B2, S2, H2, hd2 = 8, 512, 12, 64
    d2 = H2 * hd2
    rng2 = np.random.default_rng(2)
    q2, k2, v2 = (be.tensor(rng2.standard_normal(B2 * S2 * d2, dtype=np.float32))
                  for _ in range(3))
    o2, l2 = be.zeros(B2 * S2 * d2), be.zeros(S2 * H2)
    metas = [hip.FlashAttnMeta(S2, d2, hd2, 0.125, b * S2) for b in range(B2)]
    metas = [(m, be.meta(m)) for m in metas]

    def flash_all():
        for shape, meta in metas:
            be.flash_attention(q2, k2, v2, o2, l2, shape, meta)
    flash_all()
    be.synchronize()
    be.timer_start()
    for _ in range(reps):
        flash_all()
    c2_ms = be.timer_stop() / reps
    c2_flop = 2 * hd2 * S2 * (S2 + 1) * B2 * H2
    rn = prefill_rates(c2_ms, 0, c2_flop, 0, c2_flop, 0)
    bshape = hip.FlashAttnMeta(S2, d2, hd2, 0.125, 0)
    bmeta = be.meta(bshape)
    l2b = be.zeros(B2 * S2 * H2)
    be.flash_attention_batched(q2, k2, v2, o2, l2b, bshape, bmeta, B2)
    be.synchronize()
    be.timer_start()
    for _ in range(reps):
        be.flash_attention_batched(q2, k2, v2, o2, l2b, bshape, bmeta, B2)
    c2b_ms = be.timer_stop() / reps
    rb = prefill_rates(c2b_ms, 0, c2_flop, 0, c2_flop, 0)
    return {"workload": "config 2: flash attention 8 x 12 x 512 x 64 (seed 2)",
            "kernel": "split-fp16 flash (fp32-accurate; split-bf16 recompute of any tile "
                      "with an operand beyond fp16's range)", "flop": c2_flop,
            "per_node_ms": round(c2_ms, 4),
            "per_node_tflops": rn["tflops"],
            "per_node_fp32_equiv_over_fp32_peak": rn["fp32_equiv_over_fp32_peak"],
            "per_node_roofline": rn["roofline"],
            "batched_ms": round(c2b_ms, 4),
            "batched_tflops": rb["tflops"],
            "batched_fp32_equiv_over_fp32_peak": rb["fp32_equiv_over_fp32_peak"],
            "batched_roofline": rb["roofline"]}


def cpu_baseline(cfg, weights, prompt_len, budget_s=10.0, max_steps=None, threads=1):
    """The oracle's decode steps over config 4's window (positions
    prompt_len..seq_len-1, then back to prompt_len), one sequence, until
    `budget_s` seconds (or `max_steps` steps) have run.  tok/s, steps, s."""
    ora = entry.load_oracle()
    ora.set_threads(threads)
    s = ora.OracleSession(cfg, weights, cfg.seq_len)
    s.set_len(prompt_len)
    tok = 1
    t0 = time.perf_counter()
    n = 0
    window = cfg.seq_len - prompt_len
    while (max_steps is None or n < max_steps) and time.perf_counter() - t0 < budget_s:
        if n and n % window == 0:
            s.set_len(prompt_len)  # the next window
        logits = s.decode_step(tok)
        tok = ora.argmax(logits)
        n += 1
    dt = time.perf_counter() - t0
    s.close()
    ora.set_threads(1)
    return n / dt, n, dt


def cpu_baseline_sequences(cfg, weights, prompt_len, threads, budget_s=8.0):
    """All host cores the way batch-32 decode uses them: `threads` sequences
    decoded at once, one single-threaded oracle session per host thread (the
    sessions share the weights; ctypes releases the GIL for each call), each
    over config 4's window until `budget_s` seconds have run.  Aggregate
    tok/s, (mean steps per sequence, seconds)."""
    import threading
    ora = entry.load_oracle()
    ora.set_threads(1)
    sess = []
    for _ in range(threads):
        s = ora.OracleSession(cfg, weights, cfg.seq_len)
        s.set_len(prompt_len)
        sess.append(s)
    start = threading.Barrier(threads + 1)
    done = [0] * threads
    window = cfg.seq_len - prompt_len

    def run(i, s):
        start.wait()
        tok, n, t0 = 1, 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            if n and n % window == 0:
                s.set_len(prompt_len)
            tok = ora.argmax(s.decode_step(tok))
            n += 1
        done[i] = n

    ts = [threading.Thread(target=run, args=(i, s)) for i, s in enumerate(sess)]
    for t in ts:
        t.start()
    start.wait()
    t0 = time.perf_counter()
    for t in ts:
        t.join()
    dt = time.perf_counter() - t0
    for s in sess:
        s.close()
    return sum(done) / dt, sum(done) / threads, dt


def cpu_prefill_baseline(cfg, weights, tokens, threads):
    """The oracle's prefill of one prompt (the reference CPU backend's
    InferenceSession::prefill restated), tok/s."""
    ora = entry.load_oracle()
    ora.set_threads(threads)
    s = ora.OracleSession(cfg, weights, cfg.seq_len)
    t0 = time.perf_counter()
    s.prefill(tokens)
    dt = time.perf_counter() - t0
    s.close()
    ora.set_threads(1)
    return len(tokens) / dt, dt


def sampled_generate_measurement(hip, be, model, prompt, ctx, steps=64, reps=3):
    """run_chat's own loop (main.rs:162): generate(prompt, steps, 0.8, 40,
    0.95, 1.15) on every sequence from empty caches (inference.rs:264-326):
    the prefill, then `steps` rounds of sample_token over each sequence's
    history (its prompt and the tokens so far) and a decode step, all on the
    device (draws from seeded uniforms).  Per round: the generate's time less
    the same prefill timed alone (medians of `reps`)."""
    import time
    B = prompt.shape[0]
    uni = np.random.default_rng(11).random((steps, B))
    sess = hip.Session(model, ctx, B)
    args = (steps, 0.8, 40, 0.95, 1.15)
    sess.generate(prompt, *args, uniforms=uni)  # warm: captures
    gen, pre, counts = [], [], 0
    for _ in range(reps):
        sess.truncate(0)
        be.synchronize()
        t0 = time.perf_counter()
        toks = sess.generate(prompt, *args, uniforms=uni)
        gen.append(time.perf_counter() - t0)
        counts = sum(len(t) for t in toks)
        sess.truncate(0)
        be.synchronize()
        t0 = time.perf_counter()
        sess.prefill(prompt, want_logits=False)
        be.synchronize()
        pre.append(time.perf_counter() - t0)
    sess.close()
    g, p = float(np.median(gen)), float(np.median(pre))
    per = (g - p) / steps
    return {"workload": f"config 4's prompts ({B} x {prompt.shape[1]}, seed 4) through "
                        f"generate(..., {steps}, 0.8, 40, 0.95, 1.15) as run_chat calls it: "
                        f"prefill, then {steps} rounds of device sampling + decode step",
            "generate_ms": round(g * 1e3, 3), "prefill_ms": round(p * 1e3, 3),
            "ms_per_round": round(per * 1e3, 4), "tokens": int(counts),
            "tok_s": round(counts / (g - p), 1)}


def sampler_measurement(hip, be, reps=20):
    """akh_sample_rows on config 4's shape (32 rows x vocabulary 50257, logits
    N(0, 2^2), seed 0; 480 seen ids per row, as at KV 480) for run_chat's
    parameters and each feature alone, eager launches timed with events (the
    kernel alone: sample_token, sampling.rs:18-81, per row)."""
    rows, n, H = 32, 50257, 480
    rng = np.random.default_rng(0)
    logits = be.tensor((rng.standard_normal(rows * n) * 2).astype(np.float32))
    seen = be.tensor(rng.integers(0, n, rows * H, dtype=np.uint32))
    seen_len = be.tensor(np.full(rows, H, np.uint32))
    uni = be.tensor(rng.random(rows))
    out = be.zeros(rows, np.uint32)
    res = {"workload": f"{rows} rows x {n} logits, {H} seen ids per row, one launch per call"}
    for name, kw in (("run_chat", dict(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.15)),
                     ("top_k_40", dict(temperature=0.8, top_k=40)),
                     ("top_p_0.95", dict(temperature=0.8, top_p=0.95)),
                     ("temperature", dict(temperature=0.8)),
                     ("greedy", dict(temperature=0.0))):
        call = lambda: be.sample_rows(logits, rows, n, out, seen=seen, seen_stride=H,  # noqa: E731
                                      seen_len=seen_len, uniforms=uni, **kw)
        for _ in range(3):
            call()
        be.synchronize()
        be.timer_start()
        for _ in range(reps):
            call()
        res[name + "_us"] = round(be.timer_stop() / reps * 1e3, 2)
    for t in (logits, seen, seen_len, uni, out):
        t.free()
    return res


def shader_graph_measurement(pkg, hip, be, cfg, weights, session_tokens, capture=True):
    """Config 1 through the reference's per-shader decode graph: ShaderDecoder
    rebuilds build_decode_layer node for node from the C-ABI launchers (one
    launcher per shader, inference_graphs.rs:339-509), captures it once and
    replays it every step after rewriting the four dynamic metas, and reads
    the logits back, as InferenceSession::decode_step does
    (inference.rs:178-262).  As generate does on an empty cache
    (inference.rs:288-289), the 64-token prompt goes through the per-shader
    prefill graph (prefill, inference.rs:61-176, build_prefill_layer,
    inference_graphs.rs:198-337: its tensors and metas allocated as it is
    built, then run once; timed on a warm backend, whose freed tensors it
    reuses), then 64 greedy steps with the argmax on the host.
    This is what the reference's own emitter gets from the launchers, beside
    the session API's fused step."""
    import time
    dec = pkg.shader_graph.ShaderDecoder(hip, be, cfg, weights, 128, capture=capture)
    prompt = [int(t) for t in pkg.synthetic_tokens(64, cfg.vocab_size, seed=1)]
    for _ in range(2):  # warm: first launches, and the backend's tensor pool
        dec.prefill(prompt)
        dec.reset()
    pre = []
    for _ in range(3):
        be.synchronize()
        t0 = time.perf_counter()
        logits = dec.prefill(prompt)
        pre.append(time.perf_counter() - t0)
        dec.reset()
    logits = dec.prefill(prompt)
    toks = [int(np.argmax(logits))]
    t2 = time.perf_counter()
    for _ in range(64):
        logits = dec.decode_step(toks[-1])
        toks.append(int(np.argmax(logits)))
    t3 = time.perf_counter()
    replay_ms = None
    if capture:
        be.synchronize()
        be.timer_start()
        for _ in range(16):
            dec.graph.execute()
        replay_ms = be.timer_stop() / 16
    L = cfg.num_layers
    out = {"workload": "config 1 through the per-shader graphs from the C-ABI launchers: the "
                       "64-token prompt through build_prefill_layer's nodes (allocated as "
                       "built, run once; median of 3 on a warm backend), then "
                       "build_decode_layer replayed as a hipGraph with live metas; logits "
                       "read back and argmax on the host each step",
           "launches_per_step": 17 * L + 3,
           "prompt_prefill_ms": round(float(np.median(pre)) * 1e3, 3),
           "ms_per_token": round((t3 - t2) / 64 * 1e3, 3),
           "tok_s": round(64 / (t3 - t2), 1),
           "graph_replay_ms": round(replay_ms, 3) if capture else None,
           "decode": "graph replays" if capture else "eager launches (no capture)",
           "tokens_match_session": toks == session_tokens}
    dec.close()
    return out


def cpu_config1(pkg, cfg, weights, threads):
    """Config 1 in full on the oracle: prefill of the 64-token prompt
    (seed 1), then 64 greedy decode steps, each token the first maximum of
    the previous logits (InferenceSession::generate's greedy loop,
    inference.rs:264-326).  Returns the figures and the 65 greedy tokens."""
    ora = entry.load_oracle()
    ora.set_threads(threads)
    s = ora.OracleSession(cfg, weights, 128)
    prompt = pkg.synthetic_tokens(64, cfg.vocab_size, seed=1)
    t0 = time.perf_counter()
    logits = s.prefill(prompt)
    tp = time.perf_counter() - t0
    toks = [ora.argmax(logits)]
    t1 = time.perf_counter()
    for _ in range(64):
        toks.append(ora.argmax(s.decode_step(toks[-1])))
    td = time.perf_counter() - t1
    s.close()
    ora.set_threads(1)
    return {"value": round(64 / td, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_token": round(td / 64 * 1e3, 3), "prefill_s": round(tp, 3),
            "total_s": round(tp + td, 3),
            "sample": "config 1 in full: oracle prefill of the 64-token prompt (seed 1), then "
                      "64 greedy decode steps (value = decode tokens / decode time)"}, toks


def cpu_config5(cfg, weights, threads, T=2048, budget_s=10.0, max_steps=16):
    """A labelled config-5 slice on the oracle: one sequence of the scaled
    architecture decoding at KV length up to T, over a zero KV prefix (the
    cost of a step does not depend on the cached values), until `budget_s`
    seconds or `max_steps` steps have run."""
    ora = entry.load_oracle()
    ora.set_threads(threads)
    s = ora.OracleSession(cfg, weights, T)
    s.set_len(T - max_steps)
    tok, n = 1, 0
    t0 = time.perf_counter()
    while n < max_steps and time.perf_counter() - t0 < budget_s:
        tok = ora.argmax(s.decode_step(tok))
        n += 1
    dt = time.perf_counter() - t0
    s.close()
    ora.set_threads(1)
    return {"value": round(n / dt, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "steps": n, "seconds": round(dt, 2),
            "sample": f"config 5 slice: oracle decode of 1 sequence of the scaled architecture "
                      f"(bf16-valued weights, seed 5), {n} steps at KV length "
                      f"{T - max_steps + 1}..{T - max_steps + n}, zero KV prefix"}


def host_cpu():
    """(model name, logical CPUs) of the host."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return name, os.cpu_count() or 1


def cpu_limits():
    """CPUs this process may run on (affinity) and its cgroup CPU quota
    (cpu.max / cfs quota in CPUs; None when unlimited or unreadable)."""
    quota = None
    for qf, pf in (("/sys/fs/cgroup/cpu.max", None),
                   ("/sys/fs/cgroup/cpu/cpu.cfs_quota_us", "/sys/fs/cgroup/cpu/cpu.cfs_period_us")):
        try:
            if pf is None:
                q, p = open(qf).read().split()[:2]
            else:
                q, p = open(qf).read().strip(), open(pf).read().strip()
            if q not in ("max", "-1"):
                quota = round(int(q) / int(p), 2)
            break
        except (OSError, ValueError):
            continue
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    return aff, quota


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill measurement")
    ap.add_argument("--kernel-reps", type=int, default=60)
    ap.add_argument("--no-scaled", action="store_true",
                    help="skip config 5 (scaled architecture) decode and prefill")
    ap.add_argument("--no-scaled-decode", action="store_true",
                    help="measure config 5's prefill legs only")
    ap.add_argument("--prefill-only", action="store_true",
                    help="measure only config 3's prefill legs and print them (for profiling)")
    ap.add_argument("--scaled-prefill-only", action="store_true",
                    help="measure only config 5's prefill legs and print them (for profiling: "
                         "no graph replays)")
    ap.add_argument("--config2-only", action="store_true",
                    help="measure only config 2's flash legs (8 per-node launches, then the "
                         "batched launch, 10 timed rounds each) and print them (for profiling)")
    ap.add_argument("--shader-graph-only", action="store_true",
                    help="run only config 1 through the per-shader graphs and print it")
    ap.add_argument("--eager-shader", action="store_true",
                    help="with --shader-graph-only: decode steps launch eagerly instead of "
                         "replaying the captured graph (for kernel tracers)")
    ap.add_argument("--sampler-only", action="store_true",
                    help="time only the device sampler on config 4's shape and print it")
    ap.add_argument("--kernels-only", action="store_true",
                    help="run only the per-kernel decode legs, no graph replay (for counter "
                         "runs); config 5's too unless --no-scaled")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "sequences shard by data parallelism with no exchange, so N GPUs would "
              "run N independent copies of this benchmark.", file=sys.stderr)
        sys.exit(2)

    pkg = entry.load_package()
    hip = pkg.hip
    if args.sampler_only:
        be = hip.Backend(0)
        print(json.dumps({"sampler": sampler_measurement(hip, be)}), flush=True)
        be.close()
        return
    if args.scaled_prefill_only:
        be = hip.Backend(0)
        log("bench: scaled config weights (seed 5, bf16 values)")
        w5 = pkg.synthetic_weights(pkg.ModelConfig.scaled(), seed=5, bf16=True)
        print(json.dumps({"scaled": scaled_measurement(pkg, hip, be, w5, with_decode=False)}),
              flush=True)
        be.close()
        return
    cfg = pkg.ModelConfig.akasha_hall_1()
    B, P, CTX = 32, 448, 512
    log("bench: generating hall-1.0 weights (seed 0)")
    w = pkg.synthetic_weights(cfg, seed=0)
    be = hip.Backend(0)
    if args.shader_graph_only:
        out = shader_graph_measurement(pkg, hip, be, cfg, w, [], capture=not args.eager_shader)
        out.pop("tokens_match_session")
        print(json.dumps({"config1": {"shader_graph": out}}), flush=True)
        be.close()
        return
    model = hip.Model(be, cfg)
    model.upload(w)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_measurement(pkg, hip, be, model, cfg, CTX, reps=2)}),
              flush=True)
        model.close()
        be.close()
        return
    if args.config2_only:
        print(json.dumps({"config2": config2_measurement(hip, be)}), flush=True)
        model.close()
        be.close()
        return
    if args.kernels_only:
        out = kernel_legs_only(pkg, hip, be, model, cfg, args.kernel_reps, not args.no_scaled)
        print(json.dumps(out), flush=True)
        model.close()
        be.close()
        return
    sess = hip.Session(model, CTX, B)
    prompt = pkg.synthetic_tokens(B * P, cfg.vocab_size, seed=4).reshape(B, P)
    log("bench: prefill 32 x 448")
    sess.prefill(prompt, want_logits=False)
    window = CTX - P

    def run_steps(n):
        done, total_ms = 0, 0.0
        while done < n:
            k = min(window, n - done)
            sess.truncate(P)
            be.synchronize()
            be.timer_start()
            sess.decode_greedy(k, want_tokens=False)
            total_ms += be.timer_stop()
            done += k
        return total_ms

    log(f"bench: warmup {args.warmup} decode steps")
    if args.warmup:
        run_steps(args.warmup)
    # Whole 64-step windows (positions 448..511), whatever --steps asks for,
    # so the line always measures config 4's full KV range.
    windows = max(1, -(-args.steps // window))
    steps = windows * window
    log(f"bench: timing {steps} decode steps ({windows} window(s) of positions "
        f"{P}..{CTX - 1}; {args.steps} requested)")
    ms = run_steps(steps)
    ms_per_step = ms / steps
    tok_s = B * steps / (ms / 1e3)

    # Whole-step HBM roofline over the same position schedule.
    total_bytes = windows * sum(decode_step_bytes(cfg, B, P + i + 1) for i in range(window))
    step_gbs = total_bytes / (ms / 1e3) / 1e9
    launches_per_step = sess.decode_launches()

    # The same windows with each layer's residual adds + RMSNorms folded into
    # the GEMMs (five launches per layer instead of seven): not the default,
    # reported beside it.
    sess.set_fused_norm(True)
    run_steps(window)  # capture + warm
    fused_ms = run_steps(steps)
    fused_norm = {"ms_per_step": round(fused_ms / steps, 5),
                  "launches_per_step": sess.decode_launches(),
                  "step_frac": round(total_bytes / (fused_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
    sess.set_fused_norm(False)

    log("bench: sampled generate (run_chat's parameters)")
    sampled = sampled_generate_measurement(hip, be, model, prompt, CTX, steps=window)
    sampled["sampler"] = sampler_measurement(hip, be)

    # Dominant kernel: decode attention at T = 481 (pos 480), launches cycled
    # over the 12 layers so each reads its KV rows from HBM as in a step.
    sess.truncate(P)
    sess.decode_greedy(32, want_tokens=False)
    T = P + 32 + 1
    kernels, attn_dispatch_ms = decode_kernel_legs(sess, cfg, B, T, args.kernel_reps)
    kms = {n: k["ms"] for n, k in kernels.items()}
    attn_bytes = kernels["decode_attn"]["bytes"]
    attn_gbs = attn_bytes / (kms["decode_attn"] / 1e3) / 1e9

    prefill = None if args.no_prefill else prefill_measurement(pkg, hip, be, model, cfg, CTX)

    # Config 1: batch-1 greedy latency (64-token prompt, seed 1; 64 steps).
    s1 = hip.Session(model, 128, 1)
    p1 = pkg.synthetic_tokens(64, cfg.vocab_size, seed=1).reshape(1, 64)
    _, first = s1.prefill(p1, want_logits=False)
    s1.decode_greedy(8, want_tokens=False)  # capture + warm
    s1.truncate(64)
    be.synchronize()
    be.timer_start()
    s1.decode_greedy(64, want_tokens=False)
    c1_ms = be.timer_stop()
    # The same 64 steps again for their tokens (compared with the CPU leg's).
    s1.truncate(64)
    config1_tokens = [int(first[0])] + [int(t) for t in s1.decode_greedy(64)[:, 0]]
    s1.close()
    c1_bytes = decode_step_bytes(cfg, 1, 64 + 32)
    config1 = {"workload": "config 1: hall-1.0 batch 1, 64-token prompt (seed 1), 64 greedy steps",
               "ms_per_token": round(c1_ms / 64, 4), "tok_s": round(64 / (c1_ms / 1e3), 1),
               "hbm_frac": round(c1_bytes / (c1_ms / 64 / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
    log("bench: config 1 through the per-shader decode graph")
    config1["shader_graph"] = shader_graph_measurement(pkg, hip, be, cfg, w, config1_tokens)

    config2 = config2_measurement(hip, be)

    scaled, w5, c5 = None, None, pkg.ModelConfig.scaled()
    if not args.no_scaled or not args.no_cpu:
        log("bench: scaled config weights (seed 5, bf16 values)")
        w5 = pkg.synthetic_weights(c5, seed=5, bf16=True)
    if not args.no_scaled:
        scaled = scaled_measurement(pkg, hip, be, w5, with_prefill=not args.no_prefill,
                                    with_decode=not args.no_scaled_decode)

    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline (oracle decode step, 1 thread)")
        v1, n1, t1 = cpu_baseline(cfg, w, P, threads=1)
        cpu = {"value": round(v1, 3), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"oracle decode of 1 sequence, {n1} steps over config 4's window "
                         f"(positions 448..511, repeated; {t1:.1f} s), zero KV prefix; the "
                         f"reference CPU backend runs one sequence per session"}
        aff, quota = cpu_limits()
        # The box's CPU share is 16 (its OMP_NUM_THREADS), whatever nproc says.
        nt = max(1, min(16, aff, int(quota) if quota else 16))
        log(f"bench: CPU baseline ({nt} sequences at once, one thread each)")
        vN, nN, tN = cpu_baseline_sequences(cfg, w, P, nt)
        cpu_omp = {"value": round(vN, 3), "unit": "tok/s", "cores": nt, "kind": "port",
                   "sample": f"{nt} sequences decoded at once, one oracle session per host "
                             f"thread, {nN:.0f} steps each over config 4's window ({tN:.1f} s); "
                             f"batch-32 decode over all host cores"}
        # The column-split OpenMP GEMV of one sequence, for comparison: the
        # reference's per-sequence path with its matmuls spread over threads.
        vO, nO, tO = cpu_baseline(cfg, w, P, budget_s=4.0, max_steps=32, threads=nt)
        cpu_omp["one_sequence_omp"] = {"value": round(vO, 3), "threads": nt, "steps": nO,
                                       "seconds": round(tO, 2)}
        # A labelled prefill slice: config 3's sequence 0 (512 tokens).
        log(f"bench: CPU baseline (oracle prefill of 512 tokens, {nt} threads)")
        ptok = pkg.synthetic_tokens(16 * 512, cfg.vocab_size, seed=3)[:512]
        vp, tp = cpu_prefill_baseline(cfg, w, ptok, nt)
        cname, ncpu = host_cpu()
        cpu["host"] = cpu_omp["host"] = {"cpu_model": cname, "nproc": ncpu,
                                         "affinity_cpus": aff, "cgroup_cpu_quota": quota}
        cpu_omp["prefill"] = {"value": round(vp, 2), "unit": "tok/s", "cores": nt,
                              "sample": f"oracle prefill of config 3's sequence 0 (512 "
                                        f"tokens), column-split OpenMP ({tp:.1f} s)"}
        # The same prefill on one thread, over the first 64 of those tokens.
        log("bench: CPU baseline (oracle prefill of 64 tokens, 1 thread)")
        vp1, tp1 = cpu_prefill_baseline(cfg, w, ptok[:64], 1)
        cpu["prefill"] = {"value": round(vp1, 2), "unit": "tok/s", "cores": 1,
                          "sample": f"oracle prefill of the first 64 tokens of config 3's "
                                    f"sequence 0, one thread ({tp1:.1f} s)"}
        # Config 1 in full (prompt + 64 greedy steps), one thread and all.
        log("bench: CPU config 1 (64-token prefill + 64 greedy steps), 1 thread")
        c1cpu, c1toks = cpu_config1(pkg, cfg, w, 1)
        log(f"bench: CPU config 1, {nt} threads")
        c1omp, _ = cpu_config1(pkg, cfg, w, nt)
        c1cpu["tokens_match_gpu"] = c1toks == config1_tokens
        config1["cpu_baseline"] = c1cpu
        config1["cpu_baseline_omp"] = c1omp
        # A config-5 slice: one sequence of the scaled architecture at KV ~2048.
        log("bench: CPU config 5 slice (1 sequence at KV 2048), 1 thread")
        c5cpu = cpu_config5(c5, w5, 1)
        log(f"bench: CPU config 5 slice, {nt} threads")
        c5omp = cpu_config5(c5, w5, nt, budget_s=4.0, max_steps=8)
        log(f"bench: CPU config 5 prefill slice (64 tokens), {nt} threads")
        p5 = pkg.synthetic_tokens(8 * 2048, c5.vocab_size, seed=7)[:64]
        vp5, tp5 = cpu_prefill_baseline(c5, w5, p5, nt)
        c5omp["prefill"] = {"value": round(vp5, 3), "unit": "tok/s", "cores": nt,
                            "sample": f"oracle prefill of the first 64 tokens of config 5's "
                                      f"prefill sequence 0 (seed 7), column-split OpenMP "
                                      f"({tp5:.1f} s)"}
        if scaled is None:
            scaled = {}
        scaled["cpu_baseline"] = c5cpu
        scaled["cpu_baseline_omp"] = c5omp
    else:
        cpu_omp = None

    sess.close()
    model.close()
    be.close()

    out = {
        "metric": "decode tok/s @ batch 32 ctx 512 (%HBM roofline)",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"config 4: akasha-hall 1.0 greedy decode, batch 32, "
                               f"prefill 448 (seed 4), {windows} x 64 steps at positions "
                               f"{P}..{CTX - 1} (KV {P + 1}..{CTX})",
                   "model": "akasha-hall-1.0 (162M)", "global_batch": B, "seq_len": CTX,
                   "parallelism": "none (1 GPU)",
                   "launches_per_step": launches_per_step},
        "roofline": {"kernel": "decode_attn (T=481, layers cycled)", "bound": "hbm",
                     "kernel_ms": round(kms["decode_attn"], 5),
                     "dispatch_ms": round(attn_dispatch_ms, 5),
                     "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": TRAFFIC_SOURCE,
                     "algorithmic_bytes": attn_bytes},
        "step_roofline": {"achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                          "bytes_per_step_mean": int(total_bytes / steps)},
        "decode_fused_norm": fused_norm,
        "decode_sampled": sampled,
        "kernels": kernels,
        "prefill": prefill,
        "config1": config1,
        "config2": config2,
        "scaled": scaled,
        "cpu_baseline": cpu,
        "cpu_baseline_omp": cpu_omp,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
