"""Benchmark of the MI355X decode hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (BASELINE.json metric "Q4/Q2 matvec GB/s"): BASELINE config 2, the
Q2_B64 fused dequant-matvec of the FFN down-projection, 5120 x 17408, batch
1, fp16 s_in/s_out as production loads them. One step = one
ctox_hip_matrix_dispatch (one launch of the tiled matvec, which stages the
activation itself) on a resident weight copy; copies rotate over > 512 MB so the 256 MB Infinity Cache
cannot serve repeats. `value` = algorithmic bytes per step / step time.

Also reported under "extra": config 1 (Q4 17408 x 5120), config 3 (one
decoder layer's projections at M = 2/4/8 draft rows), config 4 (gated-delta
decode step and 4096-token prefill). Synthetic seeded data of the BASELINE
shapes; weights are random-init in the crate's packed layout.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ctox-llm_amd"))

HBM_PEAK_GBS = 8000.0
REPLICATES = 5
DRAFT_VOCAB = 32768
INFINITY_CACHE = 256 << 20
HEAD_KERNEL = "ctox_q2_mv_tile2x0_gfx950"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "ctox_q2_mv_tile2x0_gfx950.config2.traffic.txt")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def matvec_bytes(rows, cols, dtype, batch=1, scales=True):
    bb = 34 if dtype == 1 else 18
    b = rows * (cols // 64) * bb + batch * (cols + rows) * 4
    if scales:
        b += 2 * (cols + rows)
    return b


class Timer:
    """HIP events on the stream the kernels are launched on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch
        self.start = torch.cuda.Event(enable_timing=True)
        self.stop = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.torch.cuda.synchronize()
        self.start.record()
        return self

    def __exit__(self, *exc):
        self.stop.record()
        self.torch.cuda.synchronize()
        self.ms = self.start.elapsed_time(self.stop)


def make_matrices(hip, ctox_hip, synth, dtype, rows, cols, seed, copies):
    w = synth.random_matrix(dtype, rows, cols, seed)
    rng = np.random.default_rng(seed + 1)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    op = ctox_hip.FusedMatVec(ctox_hip.TensorDType(dtype), w, rows, cols,
                              s_in=ctox_hip.ScaleSlice.F16Le(s_in.view(np.uint8)),
                              s_out=ctox_hip.ScaleSlice.F16Le(s_out.view(np.uint8)))
    mats = [hip.prepare(op) for _ in range(copies)]
    return mats, (w, s_in, s_out)


def bench_matvec(torch, hip, ctox_hip, synth, dtype, rows, cols, xkind, steps, warmup, batch=1, seed=3):
    nbytes = rows * (cols // 64) * (34 if dtype == 1 else 18)
    copies = max(2, -(-2 * INFINITY_CACHE // nbytes))
    mats, host = make_matrices(hip, ctox_hip, synth, dtype, rows, cols, seed, copies)
    x = torch.from_numpy(synth.activation(xkind, cols, seed + 7, batch)).cuda()
    y = torch.empty((batch, rows), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for i in range(warmup):
        mats[i % copies].dispatch(x.data_ptr(), batch, y.data_ptr(), stream)
    # Five windows of `steps` dispatches each; the median window is reported.
    wins = []
    for _ in range(REPLICATES):
        with Timer(torch) as t:
            for i in range(steps):
                mats[i % copies].dispatch(x.data_ptr(), batch, y.data_ptr(), stream)
        wins.append(t.ms / steps)
    step_ms = float(np.median(wins))
    # A batch-1 step is exactly one launch of the tiled matvec kernel on the
    # timed stream, so the events around the timed region give the kernel's
    # average duration (back-to-back launches; rocprof's average of the same
    # kernel agrees).
    kernel_ms = step_ms
    b = matvec_bytes(rows, cols, dtype, batch)
    res = {"rows": rows, "cols": cols, "dtype": "q4_b64" if dtype == 1 else "q2_b64", "batch": batch,
           "copies": copies, "bytes_per_call": b, "step_us": step_ms * 1e3, "kernel_us": kernel_ms * 1e3,
           "step_us_replicates": [round(w * 1e3, 3) for w in wins],
           "step_GBps": b / (step_ms * 1e-3) / 1e9, "kernel_GBps": b / (kernel_ms * 1e-3) / 1e9}
    for m in mats:
        m.close()
    return res, host


def traffic_bytes():
    """HBM bytes per launch of the headline kernel, from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters
    on a plain copy of known size); None when no summary is present."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def copy_reference(torch, mib=256, reps=5):
    """A plain device copy of known size: the realistic HBM rate of this box
    and the calibration kernel for the FETCH_SIZE/WRITE_SIZE counters."""
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    with Timer(torch) as t:
        for _ in range(reps):
            dst.copy_(src)
    us = t.ms * 1e3 / reps
    return {"bytes_read": mib << 20, "bytes_written": mib << 20, "us": us,
            "GBps_read_plus_write": 2 * (mib << 20) / (us * 1e-6) / 1e9}


def read_floor(torch, hip, nbytes, steps=200):
    """The HBM floor of one launch: ctox_stream_read_gfx950 reading `nbytes`
    (the matvec's algorithmic bytes) with the tiled kernel's access pattern,
    rotating over copies above the Infinity Cache, median of REPLICATES
    windows of `steps` back-to-back launches. At 1 GiB per launch the
    per-launch ramp and tail vanish: the sustainable streaming read rate."""
    import ctypes
    nbytes = (nbytes + 15) // 16 * 16
    copies = max(2, -(-2 * INFINITY_CACHE // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    out = torch.empty((nbytes + 8191) // 8192, dtype=torch.int32, device="cuda")
    lib = ctox_lib()
    stream = torch.cuda.current_stream().cuda_stream

    def run(i):
        st = lib.ctox_hip_stream_read_device(hip.handle, ctypes.c_void_p(bufs[i % copies].data_ptr()), nbytes,
                                             ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream))
        if st != 0:
            raise RuntimeError("stream read failed")
    for i in range(20):
        run(i)
    wins = []
    for _ in range(REPLICATES):
        with Timer(torch) as t:
            for i in range(steps):
                run(i)
        wins.append(t.ms / steps)
    us = float(np.median(wins)) * 1e3
    return {"bytes": nbytes, "us": us, "GBps": nbytes / (us * 1e-6) / 1e9, "frac_of_8TBps": nbytes / (us * 1e-6) / 8e12}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(dtype, rows, cols, host, budget_s=12.0):
    """The crate's feature-dispatched CPU path (AVX2 restatement), one core."""
    from oracle import oracle as orc
    w, s_in, s_out = host
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    mv = orc.MatVec(dtype, w, rows, cols, x, ("f16le", s_in.view(np.uint8)), ("f16le", s_out.view(np.uint8)))
    prof = orc.AVX2 if orc.avx2_available() else orc.SCALAR
    mv.run(prof)  # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        mv.run(prof)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": matvec_bytes(rows, cols, dtype) / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{n} x {rows}x{cols} {'avx2' if prof else 'scalar'} fused matvecs on 1 host core "
                      f"({os.cpu_count()} present, {cpu_model()}), {dt * 1e3:.1f} ms each"}


def bench_gdn(torch, hip, steps):
    from ctox_hip import synth  # noqa: F401
    heads, dk, dv = 32, 128, 128
    out = {}
    rng = np.random.default_rng(0)
    for T, chunk, name in ((1, 0, "decode_step"), (4096, 64, "prefill_4096_chunk64")):
        q = torch.randn(T, heads, dk, device="cuda")
        k = torch.randn(T, heads, dk, device="cuda")
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(T, heads, dv, device="cuda")
        ld = -torch.nn.functional.softplus(torch.randn(T, heads, device="cuda"))
        be = torch.sigmoid(torch.randn(T, heads, device="cuda"))
        st = torch.zeros(heads, dk, dv, device="cuda")
        o = torch.empty(T, heads, dv, device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), ld.data_ptr(), be.data_ptr(), st.data_ptr()]
        reps = steps if T == 1 else max(1, steps // 20)
        hip.gated_delta_sequence_device(*args, T, heads, dk, dv, chunk, o.data_ptr(), s)
        with Timer(torch) as t:
            for _ in range(reps):
                hip.gated_delta_sequence_device(*args, T, heads, dk, dv, chunk, o.data_ptr(), s)
        us = t.ms * 1e3 / reps
        b = T * heads * (2 * dk + 2 * dv + 2) * 4 + 2 * heads * dk * dv * 4
        out[name] = {"tokens": T, "heads": heads, "us": us, "GBps": b / (us * 1e-6) / 1e9,
                     "tokens_per_s": T / (us * 1e-6)}
    del rng
    out.update(bench_gdn_layer_core(torch, hip, steps))
    return out


def bench_gdn_layer_core(torch, hip, steps):
    """The decode engine's GatedDeltaNet token mixer core at 27B shapes (48
    value heads over 16 key heads of 128, conv kernel 4, the engine's blocked
    state layout): conv + gates + recurrence in one launch
    (ctox_hip_gdn_fused_snap_device), one row (the plain decode step) and five
    rows with a state snapshot per row (the MTP verify pass)."""
    lib = ctox_lib()
    H, KH, D, K = 48, 16, 128, 4
    kw, vw = KH * D, H * D
    C = 2 * kw + vw
    a_off, b_off = C + vw, C + vw + H
    stride = b_off + H
    g = torch.Generator(device="cuda").manual_seed(9)
    res = {}
    for R, name in ((1, "layer_core_decode_27b"), (5, "layer_core_verify5_27b")):
        proj = torch.randn(R, stride, device="cuda", generator=g)
        conv_w = torch.randn(C, K, device="cuda", generator=g) * 0.5
        conv_in = torch.randn(C, K, device="cuda", generator=g)
        conv_out = torch.empty(R, C, K, device="cuda")
        a_log = torch.randn(H, device="cuda", generator=g) * 0.3
        dt_bias = torch.randn(H, device="cuda", generator=g) * 0.3
        ld, be = torch.empty(R, H, device="cuda"), torch.empty(R, H, device="cuda")
        ssz = H * D * D
        st_in = torch.randn(ssz, device="cuda", generator=g) * 0.1
        st_out = torch.empty(R, ssz, device="cuda")
        o = torch.empty(R, H, D, device="cuda")
        s = torch.cuda.current_stream().cuda_stream

        def run():
            st = lib.ctox_hip_gdn_fused_snap_device(hip.handle, proj.data_ptr(), stride, a_off, b_off, conv_w.data_ptr(),
                                                    conv_in.data_ptr(), conv_out.data_ptr(), C * K, K, a_log.data_ptr(),
                                                    dt_bias.data_ptr(), ld.data_ptr(), be.data_ptr(), st_in.data_ptr(),
                                                    st_out.data_ptr(), ssz, 1, R, H, KH, D, D, o.data_ptr(), s)
            if st != 0:
                raise RuntimeError(lib.ctox_hip_last_error().decode())
        run()
        with Timer(torch) as t:
            for _ in range(steps):
                run()
        us = t.ms * 1e3 / steps
        # state read once, written per snapshot; projections, conv windows, outputs
        b = ssz * 4 * (1 + R) + R * stride * 4 + 2 * C * K * 4 + R * C * K * 4 + R * vw * 4
        res[name] = {"rows": R, "value_heads": H, "key_heads": KH, "us": us, "GBps": b / (us * 1e-6) / 1e9}
    return res


def ctox_lib():
    import ctox_hip
    return ctox_hip.load_library()


def bench_token_selection(torch, hip, steps):
    """Config 5's per-step token selection: k = 4 drafts, vocab 151936, greedy
    verification and the T = 0.7 rejection-sampling accept."""
    K, V = 4, 151936
    g = torch.Generator(device="cuda").manual_seed(5)
    target = torch.randn(K, V, device="cuda", generator=g) * 2.5
    draft = target + torch.randn(K, V, device="cuda", generator=g)
    bonus = torch.randn(V, device="cuda", generator=g) * 2.5
    toks = torch.argmax(draft, dim=1).to(torch.int32)
    rng = torch.tensor([12345], dtype=torch.int64, device="cuda")
    out = torch.zeros(3 + K, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    res = {}
    for name, fn in (("verify_greedy_k4", lambda: hip.verify_greedy_mtp_device(
                          draft.data_ptr(), target.data_ptr(), bonus.data_ptr(), K, V, out.data_ptr(), s)),
                     ("mtp_accept_t0.7_k4", lambda: hip.mtp_accept_device(
                          draft.data_ptr(), target.data_ptr(), bonus.data_ptr(), toks.data_ptr(), K, V, 0.7,
                          rng.data_ptr(), out.data_ptr(), s)),
                     ("sample_topk40_topp0.95_t0.8", lambda: ctox_lib().ctox_hip_sample_topk_topp_device(
                          hip.handle, bonus.data_ptr(), V, 0.8, 40, 0.95, 0.37, out.data_ptr(), s))):
        fn()
        with Timer(torch) as t:
            for _ in range(steps):
                fn()
        res[name] = {"us": t.ms * 1e3 / steps, "vocab": V, "drafts": K}
    return res


def bench_paged_attention(torch, hip, steps, tokens=32768):
    """Config 5's full-attention read: 24 query heads over 4 KV heads of 256,
    `tokens` cached at page size 16 with the crate's 128-sink / 256-recent Q4
    policy (older pages Q2), for the 1-row decode and the 5-row MTP verify."""
    from ctox_hip.paged_kv import DevicePagedKvCache
    qh, kvh, hd = 24, 4, 256
    cache = DevicePagedKvCache(hip, tokens, kvh, hd, page_tokens=16, sink_tokens=128, recent_tokens=256)
    g = torch.Generator(device="cuda").manual_seed(7)
    for i in range(0, tokens, 4096):
        n = min(4096, tokens - i)
        cache.push(torch.randn(n, kvh * hd, device="cuda", generator=g),
                   torch.randn(n, kvh * hd, device="cuda", generator=g))
    kv_bytes = cache.q2_tokens() * cache.q2_token_bytes + cache.q4_tokens() * cache.q4_token_bytes
    res = {"tokens": tokens, "page_tokens": 16, "q2_tokens": cache.q2_tokens(), "q4_tokens": cache.q4_tokens()}
    for rows in (1, 5):
        q = torch.randn(rows, qh, hd, device="cuda", generator=g)
        out = torch.empty(rows, qh, hd, device="cuda")
        cache.attention(q, rows, qh, out)
        n = max(10, steps // 4)
        with Timer(torch) as t:
            for _ in range(n):
                cache.attention(q, rows, qh, out)
        us = t.ms * 1e3 / n
        flops = 4.0 * qh * rows * tokens * hd
        res[f"rows{rows}"] = {"us": us, "kv_bytes": kv_bytes, "GBps": kv_bytes / (us * 1e-6) / 1e9,
                              "TFLOPs": flops / (us * 1e-6) / 1e12}
    return res


def bench_verify_layer(torch, hip, ctox_hip, synth, batch, steps):
    """Config 3: every projection of one decoder layer (q at the crate's
    12288 rows, k, v, o, gate, up as Q4; down as Q2) on `batch` rows."""
    tot_b, tot_us = 0, 0.0
    for name, dt, r, c in [("q", 1, 12288, 5120), ("k", 1, 1024, 5120), ("v", 1, 1024, 5120),
                           ("o", 1, 5120, 6144), ("gate", 1, 17408, 5120), ("up", 1, 17408, 5120),
                           ("down", 0, 5120, 17408)]:
        res, _ = bench_matvec(torch, hip, ctox_hip, synth, dt, r, c, "normal", max(20, steps // 4), 5, batch=batch)
        tot_b += res["bytes_per_call"]
        tot_us += res["step_us"]
    return {"us": tot_us, "GBps": tot_b / (tot_us * 1e-6) / 1e9}


def bench_decode_27b(torch, hip, steps, context=32768):
    """Config 5: the device engine on the 27B shapes (64 layers, 48 GatedDeltaNet
    and 16 full attention, Q4 projections and LM head, Q2 down projections,
    vocab 151936), paged KV page 16 with `context` random tokens; plain
    batch-1 decode and MTP k = 4 at T = 0.7 (seeded Pcg32) and greedy (T = 0,
    the crate's mode). Weights are synthetic, so draft acceptance reflects
    random heads."""
    import time
    from ctox_hip.engine import Engine, EngineConfig
    cfg = EngineConfig.qwen38_27b(max_tokens=context + 1280)
    eng = Engine(hip, cfg, seed=5)
    eng.fill_context(context, seed=9)
    q4 = (48 * (16480 * 5120 + 5120 * 6144) + 16 * (14336 * 5120 + 5120 * 6144) + 64 * 34816 * 5120
          + 151936 * 5120) * 34 // 64
    q2 = 64 * 5120 * 17408 * 18 // 64
    tok = 1234
    for _ in range(3):
        eng.decode(tok)
    n = max(10, min(steps, 40))
    t0 = time.time()
    for _ in range(n):
        eng.decode(tok)
    plain = (time.time() - t0) / n
    res = {"context": context, "page_tokens": 16, "weight_bytes_per_token": q4 + q2,
           "plain_ms_per_token": plain * 1e3, "plain_tokens_per_s": 1.0 / plain,
           "plain_weight_GBps": (q4 + q2) / plain / 1e9, "steps": n}

    # More speculative steps than plain ones: the accepted-draft count per
    # step is a random variable whose mean the tokens/s figure depends on.
    n_mtp = max(10, min(steps, 100))

    def mtp_run(tag, tok, temperature=0.7):
        eng.set_rng(0x5EED)
        tokens = 0
        eng.mtp_step(tok, temperature)  # warm
        t0 = time.time()
        for _ in range(n_mtp):
            nxt, acc = eng.mtp_step(tok, temperature)
            tokens += 1 + len(acc)
            tok = nxt
        torch.cuda.synchronize()  # the last step's commit may still be queued
        mtp = time.time() - t0
        key = "mtp_k4_greedy" if temperature == 0.0 else f"mtp_k4_T0.7{tag}"
        tag = "_greedy" if temperature == 0.0 else tag
        res[f"{key}_ms_per_step"] = mtp / n_mtp * 1e3
        res[f"mtp{tag}_tokens_per_s"] = tokens / mtp
        res[f"mtp{tag}_accepted_drafts_per_step"] = tokens / n_mtp - 1
        res[f"mtp{tag}_steps"] = n_mtp
        return tok

    tok = mtp_run("", tok)
    # The crate's own speculative mode: greedy drafts and prefix-match verify.
    tok = mtp_run("", tok, temperature=0.0)
    # The release-bound draft vocabulary (Q/src/decoder.rs:589-627): a seeded
    # 32768-token subset here (random weights: no trained coverage).
    ids = np.sort(np.random.default_rng(3).choice(cfg.vocab_size, DRAFT_VOCAB, replace=False)).astype(np.uint32)
    eng.set_draft_vocab(ids)
    res["draft_vocab"] = DRAFT_VOCAB
    mtp_run("_restricted", tok)
    eng.close()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only")
    ap.add_argument("--only", choices=["decode", "attention", "gdn", "selection", "verify", "config1", "config2",
                                       "floor"],
                    help="run one extra workload alone and print its result (for profiling)")
    ap.add_argument("--context", type=int, default=32768, help="context of --only decode / attention")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import ctox_hip
    from ctox_hip import synth

    hip = ctox_hip.HipBackend(0)
    log("backend", hip.kind(), hip.profile(), torch.cuda.get_device_name(0))
    if args.only:
        res = {"decode": lambda: bench_decode_27b(torch, hip, args.steps, args.context),
               "attention": lambda: bench_paged_attention(torch, hip, args.steps, args.context),
               "gdn": lambda: bench_gdn(torch, hip, args.steps),
               "selection": lambda: bench_token_selection(torch, hip, args.steps),
               "verify": lambda: bench_verify_layer(torch, hip, ctox_hip, synth, 5, args.steps),
               "config1": lambda: bench_matvec(torch, hip, ctox_hip, synth, 1, 17408, 5120, "normal", args.steps,
                                               args.warmup)[0],
               "config2": lambda: bench_matvec(torch, hip, ctox_hip, synth, 0, 5120, 17408, "swiglu", args.steps,
                                               args.warmup)[0],
               "floor": lambda: {"config2_bytes": read_floor(torch, hip, matvec_bytes(5120, 17408, 0), args.steps),
                                 "config1_bytes": read_floor(torch, hip, matvec_bytes(17408, 5120, 1), args.steps),
                                 "sustained_1GiB": read_floor(torch, hip, 1 << 30, 20)}
               }[args.only]()
        print(json.dumps({"only": args.only, "result": res}), flush=True)
        return

    head, host2 = bench_matvec(torch, hip, ctox_hip, synth, 0, 5120, 17408, "swiglu", args.steps, args.warmup)
    log("config2", head)
    extra = {"config2_q2_down": head}
    if not args.quick:
        c1, _ = bench_matvec(torch, hip, ctox_hip, synth, 1, 17408, 5120, "normal", args.steps, args.warmup)
        log("config1", c1)
        extra["config1_q4_up"] = c1
        for batch in (2, 4, 8):
            extra[f"config3_verify_layer_M{batch}"] = bench_verify_layer(torch, hip, ctox_hip, synth, batch, args.steps)
            log("config3", batch, extra[f"config3_verify_layer_M{batch}"])
        extra["config4_gated_delta"] = bench_gdn(torch, hip, args.steps)
        log("config4", extra["config4_gated_delta"])
        extra["config5_token_selection"] = bench_token_selection(torch, hip, args.steps)
        log("config5", extra["config5_token_selection"])
        extra["config5_paged_attention"] = bench_paged_attention(torch, hip, args.steps)
        log("config5 attention", extra["config5_paged_attention"])
        extra["config5_decode_27b"] = bench_decode_27b(torch, hip, args.steps)
        log("config5 decode", extra["config5_decode_27b"])

    extra["copy_reference"] = copy_reference(torch)
    extra["read_floor"] = {"config2_bytes": read_floor(torch, hip, matvec_bytes(5120, 17408, 0), args.steps),
                           "config1_bytes": read_floor(torch, hip, matvec_bytes(17408, 5120, 1), args.steps),
                           "sustained_1GiB": read_floor(torch, hip, 1 << 30, 20)}
    log("read floor", extra["read_floor"])
    log("copy", extra["copy_reference"])
    cpu = None if args.no_cpu else cpu_baseline(0, 5120, 17408, host2)
    line = {
        "metric": "Q4/Q2 matvec GB/s (% of HBM peak); 27B batch-1 decode tokens/s with MTP",
        "value": round(head["step_GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["step_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q2_b64 codes, int8 MFMA, f32 accumulate/epilogue",
        "data": "synthetic (seeded; codes uniform, fp16 scales |N(0,0.02)|, x = SiLU(N)*N)",
        "config": {"workload": "config2: Q2_B64 fused dequant-matvec 5120x17408 (FFN down), batch 1, "
                               "fp16 s_in/s_out", "rows": 5120, "columns": 17408, "batch": 1,
                   "weight_copies": head["copies"],
                   "timing": f"median of {REPLICATES} windows of `steps` dispatches"},
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_GBps"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["kernel_GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(),
                     "kernel": HEAD_KERNEL, "kernel_us": round(head["kernel_us"], 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
