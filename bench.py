"""Benchmark of the INT8 GDN decode path on one MI355X.

Workload (config 1): GDN layer, B = 64 rows, HV = 32 value heads sharing H = 16 key heads, K = V = 128, window W = 64,
R = 4 Compensator Tokens, int8 state + fp32 scales; every call = decode step + end-of-window flush (the flush does work
on one call in 64).  Synthetic inputs with the config-0 distributions (q, k ~ N(0,1) l2-normalised, v ~ N(0,1), log-gate
g ~ U(-0.1, 0), beta = sigmoid(N(0,1)); states N(0, 0.02^2) quantised once), resident in HBM before timing.

Measurement:
  * `value` = amortised microseconds per decode call (step + flush, flushes included), from HIP events around graph
    replays of the decode loop.  The loop rotates NSET disjoint slot sets (> 1 GB of state) so the 256 MB MALL
    cannot hold the working set between uses of a set, and times whole rotations (every set's windows from empty
    through the all-due flush): --steps / --warmup are rounded up to rotations of 64 * NSET calls, and `steps` /
    `warmup` report the calls actually run (the warm-up, at least two rotations, is queued directly before the timed
    calls so that the GPU does not idle between them).  `achieved_gbps` divides the algorithmic bytes of those calls by their time.
    `value_spread`: the same figure for each of 9 further rotations (median, p10, p90, min, max).
  * `cpu_baseline`: the numpy oracle on config 0, its independent heads split over the host's cores (forked before the
    GPU is touched).
  * `roofline`: the timed region runs one kernel per call -- the GQA-2 step that also flushes the heads whose window it
    fills (lq_gdn_decode) -- so its achieved rate is the algorithmic bytes of the timed calls (step bytes at each fill,
    plus one all-due flush per set and window) over the timed region.  `step_roofline`: the step alone
    (lq_gdn_step), algorithmic bytes per launch over the average launch duration, from HIP events around graph replays
    of step launches over the same rotated sets (every window runs h = 0..63).  `traffic`: the HBM bytes per launch that
    rocprofv3's FETCH_SIZE / WRITE_SIZE counters read for this same command, calibrated on the 64 MiB copies it ends with.
  * the same step on a dense bf16 state (`lq_dense_step`, tuned as the INT8 step is) as the baseline, beside the
    ceiling of its access pattern (`bf16_state_rmw_ceiling`: a pure read-and-write-back stream of the same blocks).
Usage: python bench.py [--gpus 1] [--steps 1024] [--warmup 128] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

T_START = time.perf_counter()
ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "int8 GDN/KDA decode-step µs + achieved HBM GB/s at B=64,H=32,d=128"
DECODE_KERNEL = "gdn_step_kernel<128, 128, 2, false, true, 4, false>"  # lq_gdn_decode at GQA 2: step + flush of its due heads
STEP_KERNEL = "gdn_step_kernel<128, 128, 2, false, false, 4, false>"   # the step alone (lq_gdn_step)
HBM_PEAK_GBPS = 8000.0


def step_bytes(N, HV, H, K, V, R, h, bits=8):
    """Algorithmic bytes of one GDN step launch with h valid window entries per head (layout-independent minimum):
    per value head codes, Sk/Sv, U^T|Q^T, v/o/u-append, scalars, buffered u_j and w_j; per key head q/k in, k append,
    buffered k_j."""
    return N * (HV * (V * K * bits // 8 + 4 * (K + V) + 2 * R * (K + V) + 6 * V + 20 + (2 * V + 4) * h)
                + H * (6 * K + 2 * K * h))


def flush_bytes(N, HV, H, K, V, R, W, bits=8):
    """Algorithmic bytes of one flush launch on which every head of the N rows is due."""
    return N * (HV * (2 * (V * K * bits // 8 + 4 * (K + V) + 2 * R * (K + V)) + W * (2 * V + 4)) + H * W * 2 * K)


def dense_bytes(N, HV, H, K, V, elem=2):
    return N * (HV * (2 * elem * V * K + 4 * V + 4) + H * 4 * K)


def kda_step_bytes(N, HV, K, V, R, h):
    """Algorithmic bytes of one KDA step launch (HV = H) with h valid window entries per head: per (row, head) codes,
    Sk/Sv, U^T|Q^T, v in / o out / u append, the per-channel gate (a in, dt_bias in, P read + write, e_h append),
    q/k in, k append, scalars, and per window entry u_j, k_j, e_j, w_j."""
    return N * HV * (V * K + 4 * (K + V) + 2 * R * (K + V) + 4 * V + 4 * K + (2 * V + 4 * K + 4) + 2 * K + 2 + 8 * K + 8
                     + (2 * V + 4 * K + 4) * h)


def quantize_bytes(n_heads, K, V):
    """One standalone quantize: the fp32 state in, the checkpoint (codes, scales, factors) out."""
    return n_heads * (4 * V * K + V * K + 4 * (K + V) + 2 * 4 * (K + V))


def progress(msg):
    """One line per finished stage on stderr (the result stays the only line on stdout)."""
    print("[bench] %s (%.0f s)" % (msg, time.perf_counter() - T_START), file=sys.stderr, flush=True)


def event_ms(torch, stream, fn, reps):
    """Average duration of fn() (work on `stream`), from HIP events on that stream.  A spin kernel (~1 ms) queued ahead
    of the start event keeps the GPU busy while the host enqueues fn()'s launches, so that the events bracket the GPU's
    work and not the host's launch latency (which a single eager launch would otherwise add, ~20-30 us here)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()                                  # warm-up replays (default stream) done
    with torch.cuda.stream(stream):
        torch.cuda._sleep(2_000_000)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def kda_bench(torch, dev, stream, capture):
    """KDA decode (per-channel gate, Kimi form), B = 128, HV = H = 32, d = 128, W = 64, R = 4, int8
    state; 4 rotated slot sets (> 1 GB).  Returns the amortised decode call (step + flush), the step alone (mean over
    h = 0..63) and the flush with every head due."""
    from leapquant_amd.state import LeapQuantState
    B, HV, H, K, V, L, R = 128, 32, 32, 128, 128, 64, 4
    NSET = 4
    NS = B * NSET + 1
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    ssm = torch.empty(NS, HV, V, K, device=dev)
    ssm.normal_(0.0, 0.02, generator=g)
    lq = LeapQuantState(ssm, H, kda=True, L=L, R=R)
    lq.quantize(ssm, torch.arange(1, NS, device=dev, dtype=torch.int32))
    sets = [torch.arange(1 + B * k, 1 + B * (k + 1), device=dev, dtype=torch.int32) for k in range(NSET)]
    pool = []
    for _ in range(8):
        q = torch.randn(B, H, K, device=dev, generator=g)
        k = torch.randn(B, H, K, device=dev, generator=g)
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(B, HV, V, device=dev, generator=g)
        mixed = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], 1).to(torch.bfloat16).contiguous()
        gl = (-0.1 * torch.rand(B, HV * K, device=dev, generator=g)).clamp(max=-1e-4)
        a = torch.log(torch.expm1(-gl)).to(torch.bfloat16)       # -softplus(a) = g (A_log = 0, dt_bias = 0)
        b = torch.randn(B, HV, device=dev, generator=g).to(torch.bfloat16)
        pool.append((mixed, a, b))
    A_log = torch.zeros(HV, device=dev)
    dt_bias = torch.zeros(HV * K, device=dev)
    out = torch.empty(B, HV, V, device=dev, dtype=torch.bfloat16)
    vw = lq.views(ssm)

    def decode(i):
        mixed, a, b = pool[i % 8]
        lq.decode(ssm, mixed, a, b, A_log, dt_bias, sets[i % NSET], out)

    def step_only(i):
        mixed, a, b = pool[i % 8]
        lq.kstep(vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gbuf, lq.hcnt, mixed,
                 a.reshape(B, HV, K), b, A_log, dt_bias, vw["uq"], sets[i % NSET], out)

    def flush_only(kk):
        lq.kflush(vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gbuf, lq.hcnt,
                  vw["sq16"], vw["uq"], lq.Q0, sets[kk])

    CH = 64
    gdec = capture(decode, CH)
    for _ in range(2):
        gdec.replay()
    torch.cuda.synchronize()
    decode_us = event_ms(torch, stream, gdec.replay, 8) * 1e3 / CH
    # step alone: a graph of 64 steps gives each set 16; four replays take every window from h = 0 to h = 64, after
    # which every head is due and the flush graphs reset them
    lq.quantize(ssm, torch.arange(1, NS, device=dev, dtype=torch.int32))
    gst = capture(step_only, CH)
    gfl = [capture(lambda i, kk=kk: flush_only(kk), 1) for kk in range(NSET)]
    torch.cuda.synchronize()
    st_ms, fl_ms = [], []
    for r in range(3):
        st_ms.append(event_ms(torch, stream, gst.replay, 64 // (CH // NSET)))
        for kk in range(NSET):
            fl_ms.append(event_ms(torch, stream, gfl[kk].replay, 1))
    step_us = sum(st_ms[1:]) / len(st_ms[1:]) * 1e3 / CH
    flush_us = sum(fl_ms[NSET:]) / len(fl_ms[NSET:]) * 1e3
    # the KDA prefill round trip of one slot set (B x HV heads): dequant (fp32 state with the decayed window) and the
    # checkpoint (three subspace rounds, residual codes, window reset)
    rt_d, rt_q = [], []
    for r in range(3):
        rt_d.append(event_ms(torch, stream, lambda: lq.dequantize(ssm, sets[0]), 1))
        rt_q.append(event_ms(torch, stream, lambda: lq.quantize(ssm, sets[0]), 1))
    bytes_step = sum(kda_step_bytes(B, HV, K, V, R, h) for h in range(L)) / L
    # a pure loader of the same traffic (per (row, head) the step's mean bytes, writes included, as one contiguous run
    # from the head's 64 KiB block; two heads per 256-thread workgroup; the same rotated sets)
    blk = ssm.stride(1) * 4
    per_head = (int(bytes_step) // (B * HV) + 15) // 16 * 16
    sink = torch.empty(B * HV * 256, dtype=torch.int32, device=dev)
    bases = [ssm.data_ptr() + (1 + B * kk) * HV * blk for kk in range(NSET)]
    loader_us = min(probe_read_us(torch, stream, capture, bases, blk, per_head, B * HV, 2, nt, sink) for nt in (0, 1))
    res = {"workload": "KDA decode, BASELINE config 2: B=128, HV=H=32, d=128, W=64, R=4, int8 state, %d rotated slot "
                       "sets" % NSET,
           "decode_us": round(decode_us, 3), "step_us": round(step_us, 3),
           "step_gbps": round(bytes_step / (step_us * 1e-6) / 1e9, 1), "step_bytes_per_launch": int(bytes_step),
           "loader_us": round(loader_us, 3), "loader_gbps": round(bytes_step / (loader_us * 1e-6) / 1e9, 1),
           "flush_due_us": round(flush_us, 2),
           "prefill_dequant_us": round(sum(rt_d[1:]) / 2 * 1e3, 1),
           "prefill_checkpoint_us": round(sum(rt_q[1:]) / 2 * 1e3, 1)}
    del gdec, gst, gfl, lq, ssm
    torch.cuda.empty_cache()
    return res


def head_dims_bench(torch, dev, stream, capture):
    """GDN head-dim variants (K, V) = (64, 128), (64, 64) (reference kernels.py:62-65) at config 1's batch and heads
    (B = 64, HV = 32, H = 16) and the reference's window for these shapes, W = 16 (R = 4), int8 state, 4 rotated slot
    sets.  Per shape: the amortised decode call (step + flush), the step alone (mean over h = 0..15) with its
    algorithmic GB/s, a pure streaming loader of the same bytes (the latency-and-launch ceiling of a one-round kernel
    of this size), the flush with every head of a set due, and the standalone quantize of a set's fp32 states."""
    from leapquant_amd.state import LeapQuantState
    B, HV, H, L, R, NSET = 64, 32, 16, 16, 4, 4
    NS = B * NSET + 1
    res = {"workload": "GDN decode, B=64, HV=32 value / H=16 key heads, W=16, R=4, int8 state, %d rotated slot sets"
                       % NSET}
    for K, V in ((64, 128), (64, 64)):
        g = torch.Generator(device=dev)
        g.manual_seed(1005 + K + V)
        ssm = torch.empty(NS, HV, V, K, device=dev)
        ssm.normal_(0.0, 0.02, generator=g)
        lq = LeapQuantState(ssm, H, L=L, R=R)
        lq.quantize(ssm, torch.arange(1, NS, device=dev, dtype=torch.int32))
        sets = [torch.arange(1 + B * k, 1 + B * (k + 1), device=dev, dtype=torch.int32) for k in range(NSET)]
        pool = []
        for _ in range(8):
            q = torch.randn(B, H, K, device=dev, generator=g)
            k = torch.randn(B, H, K, device=dev, generator=g)
            q = q / q.norm(dim=-1, keepdim=True)
            k = k / k.norm(dim=-1, keepdim=True)
            v = torch.randn(B, HV, V, device=dev, generator=g)
            mixed = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], 1).to(torch.bfloat16).contiguous()
            gl = (-0.1 * torch.rand(B, HV, device=dev, generator=g)).clamp(max=-1e-4)
            a = torch.log(torch.expm1(-gl)).to(torch.bfloat16)
            b = torch.randn(B, HV, device=dev, generator=g).to(torch.bfloat16)
            pool.append((mixed, a, b))
        A_log = torch.zeros(HV, device=dev)
        dt_bias = torch.zeros(HV, device=dev)
        out = torch.empty(B, HV, V, device=dev, dtype=torch.bfloat16)
        vw = lq.views(ssm)

        def decode(i):
            mixed, a, b = pool[i % 8]
            lq.decode(ssm, mixed, a, b, A_log, dt_bias, sets[i % NSET], out)

        def step_only(i):
            mixed, a, b = pool[i % 8]
            lq.kstep(vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.hcnt, mixed, a,
                     b, A_log, dt_bias, vw["uq"], sets[i % NSET], out)

        def flush_only(kk):
            lq.kflush(vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gd, lq.hcnt,
                      vw["sq16"], vw["uq"], lq.Q0, sets[kk])

        CH = NSET * L                                   # one graph: every set's window from h = 0 to full
        gdec = capture(decode, CH)
        for _ in range(2):
            gdec.replay()
        torch.cuda.synchronize()
        decode_us = event_ms(torch, stream, gdec.replay, 8) * 1e3 / CH
        lq.quantize(ssm, torch.arange(1, NS, device=dev, dtype=torch.int32))
        gst = capture(step_only, CH)
        gfl = [capture(lambda i, kk=kk: flush_only(kk), 1) for kk in range(NSET)]
        torch.cuda.synchronize()
        st_ms, fl_ms = [], []
        for r in range(4):                              # step graph (every window to full), then every set's flush
            st_ms.append(event_ms(torch, stream, gst.replay, 1))
            for kk in range(NSET):
                fl_ms.append(event_ms(torch, stream, gfl[kk].replay, 1))
        step_us = sum(st_ms[1:]) / len(st_ms[1:]) * 1e3 / CH
        flush_us = sum(fl_ms[NSET:]) / len(fl_ms[NSET:]) * 1e3
        bytes_step = sum(step_bytes(B, HV, H, K, V, R, h) for h in range(L)) / L
        # a pure loader of the same traffic at this shape: per (row, value head), as many bytes as the step moves per
        # head (its mean over the window, writes included), read as one contiguous run from the head's checkpoint
        # block, two heads per 256-thread workgroup, over the same rotated sets; the faster of plain / non-temporal
        blk = ssm.stride(1) * 4
        per_head = (int(bytes_step) // (B * HV) + 15) // 16 * 16
        sink = torch.empty(B * HV * 256, dtype=torch.int32, device=dev)
        bases = [ssm.data_ptr() + (1 + B * kk) * HV * blk for kk in range(NSET)]
        loader_us = min(probe_read_us(torch, stream, capture, bases, blk, per_head, B * HV, 2, nt, sink)
                        for nt in (0, 1))
        # the standalone quantize of one set's fp32 states (B x HV heads), sets rotated
        q_ms = []
        for r in range(2 * NSET):
            ssm[1 + B * (r % NSET): 1 + B * (r % NSET + 1)].normal_(0.0, 0.02, generator=g)
            torch.cuda.synchronize()                    # the refill (default stream) before the timed quantize
            q_ms.append(event_ms(torch, stream, lambda kk=r % NSET: lq.quantize(ssm, sets[kk]), 1))
        quant_us = sum(q_ms[NSET:]) / NSET * 1e3
        qbytes = B * HV * (V * K * 4 + V * K + 4 * (K + V) + 2 * R * (K + V))
        res["K%d_V%d" % (K, V)] = {"decode_us": round(decode_us, 3), "step_us": round(step_us, 3),
                                   "step_gbps": round(bytes_step / (step_us * 1e-6) / 1e9, 1),
                                   "step_bytes_per_launch": int(bytes_step),
                                   "loader_us": round(loader_us, 3),
                                   "loader_gbps": round(bytes_step / (loader_us * 1e-6) / 1e9, 1),
                                   "flush_due_us": round(flush_us, 2),
                                   "quantize_us": round(quant_us, 2),
                                   "quantize_gbps": round(qbytes / (quant_us * 1e-6) / 1e9, 1)}
        del gdec, gst, gfl, lq, ssm
        torch.cuda.empty_cache()
    return res


def flush_quantize_bench(torch, dev, stream):
    """standalone flush and quantize of 256 x 32 heads of 128 x 128 fp32 states with Student-t
    (nu = 3, scale 0.02) entries; the flush with a full window (64 buffered entries) on every head; INT8 and 6-bit."""
    from leapquant_amd import kernels as KN
    from leapquant_amd.state import LeapQuantState
    NSL, HV, H, K, V, L, R = 256, 32, 16, 128, 128, 64, 4
    NS = NSL + 1
    g = torch.Generator(device=dev)
    g.manual_seed(1003)
    S0 = torch.empty(NS, HV, V, K, device=dev)
    for s0 in range(0, NS, 32):                      # Student-t(3) = z / sqrt(chi2_3 / 3), in chunks
        sl = slice(s0, min(NS, s0 + 32))
        z = torch.randn(S0[sl].shape, device=dev, generator=g)
        c2 = sum(torch.randn(S0[sl].shape, device=dev, generator=g) ** 2 for _ in range(3))
        S0[sl] = 0.02 * z / torch.sqrt(c2 / 3.0)
    del z, c2
    ssm = S0.clone()
    slots = torch.arange(1, NS, device=dev, dtype=torch.int32)
    nheads = NSL * HV
    res = {"workload": "BASELINE config 3: 256 x 32 heads of 128 x 128 fp32 states, Student-t(3) x 0.02; flush with "
                       "64 buffered entries on every head; value heads share a key head's window keys (GQA 2, "
                       "H = 16) or each state has its own window (gqa1: H = 32, the survey's per-head byte count)"}
    for qmax, tag, H in ((127.0, "int8", 16), (31.0, "6bit", 16), (127.0, "int8_gqa1", 32)):
        lq = LeapQuantState(ssm, H, L=L, R=R, qmax=qmax)
        vw = lq.views(ssm)
        quant = KN.make_quantize(NS, HV, K, V, L, ssm.stride(0), R=R, qmax=qmax)

        def qrun():
            quant(ssm, vw["Sq"], vw["Sk"], vw["Sv"], vw["uq"], lq.Wbuf, lq.Pbuf, lq.hcnt, lq.Q0, slots)

        ts = []
        for r in range(3 if H == 16 else 1):         # gqa1: the same states, checkpointed for its flush only
            ssm.copy_(S0)                            # the quantize overwrites its input with the checkpoint
            torch.cuda.synchronize()
            ts.append(event_ms(torch, stream, qrun, 1))
        q_us = sum(ts[1:]) / 2 * 1e3 if H == 16 else None
        if tag == "int8":
            # the prefill dequant of the same heads (window empty after the quantize): 19 KiB in, 64 KiB out per head;
            # then the checkpoints again for the flush below
            td = []
            for r in range(3):
                torch.cuda.synchronize()
                td.append(event_ms(torch, stream, lambda: lq.dequantize(ssm, slots), 1))
                ssm.copy_(S0)
                qrun()
            res["dequant_int8_us"] = round(sum(td[1:]) / 2 * 1e3, 1)
            res["dequant_int8_gbps"] = round(quantize_bytes(nheads, K, V) / (res["dequant_int8_us"] * 1e-6) / 1e9, 1)
        # a full window on every head: unit keys, values, gate products of U(-0.1, 0) log-gates
        lq.Kbuf.copy_(torch.nn.functional.normalize(torch.randn(lq.Kbuf.shape, device=dev, generator=g), dim=-1))
        lq.Ubuf.normal_(0.0, 0.02, generator=g)
        lg = -0.1 * torch.rand(NS, HV, L, device=dev, generator=g)
        w0 = torch.exp(torch.flip(torch.cumsum(torch.flip(lg, [2]), 2), [2]) - lg)   # prod of the later entries' gates
        p0 = torch.exp(lg.sum(-1, keepdim=True))

        def frun():
            lq.kflush(vw["q32"], vw["Sk"], vw["Sv"], vw["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gd, lq.hcnt,
                      vw["sq16"], vw["uq"], lq.Q0, slots)

        tf = []
        for r in range(3):
            lq.Wbuf.copy_(w0)
            lq.Pbuf.copy_(p0)
            lq.hcnt.fill_(L)
            torch.cuda.synchronize()
            tf.append(event_ms(torch, stream, frun, 1))
        f_us = sum(tf[1:]) / 2 * 1e3
        fb = flush_bytes(NSL, HV, H, K, V, R, L)
        if q_us is not None:
            res["quantize_%s_us" % tag] = round(q_us, 1)
            res["quantize_%s_gbps" % tag] = round(quantize_bytes(nheads, K, V) / (q_us * 1e-6) / 1e9, 1)
        res["flush_%s_us" % tag] = round(f_us, 1)
        res["flush_%s_bytes" % tag] = fb
        res["flush_%s_gbps" % tag] = round(fb / (f_us * 1e-6) / 1e9, 1)
        del lq, vw
    del S0, ssm
    torch.cuda.empty_cache()
    return res


def probe_read_us(torch, stream, capture, bases, stride, nbytes, nblk, per_wg, nt, sink):
    """µs per launch of leapquant_amd/_build/liblq_probe.so's streaming read: bytes [0, nbytes) of nblk blocks
    `stride` apart from bases[i % len(bases)] (launch i), per_wg blocks per 256-thread workgroup, plain (nt = 0) or
    non-temporal 16-byte loads; graphs of 64 launches, HIP events over whole rotations of the bases."""
    import ctypes
    probe = ctypes.CDLL(os.path.join(ROOT, "leapquant_amd", "_build", "liblq_probe.so"))
    probe.lq_probe_read.restype = ctypes.c_int
    probe.lq_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    NSET = len(bases)

    def launch(i):
        rc = probe.lq_probe_read(ctypes.c_void_p(bases[i % NSET]), stride, nbytes, nblk, per_wg, nt,
                                 ctypes.c_void_p(sink.data_ptr()),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc:
            raise RuntimeError("lq_probe_read failed (%d)" % rc)
    gr = capture(launch, 64)
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = NSET // 2 if NSET >= 2 else 1
    torch.cuda.synchronize()                                  # warm-up replays (default stream) done
    with torch.cuda.stream(stream):
        torch.cuda._sleep(2_000_000)                # keeps the GPU busy while the host enqueues
        e0.record(stream)
        for _ in range(reps):
            gr.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (64 * reps)


def loader_ceiling(torch, dev, stream, ssm, B, HV, NSET, R, capture):
    """What the memory system delivers to a pure streaming read of the step's own byte pattern, over the same rotated
    slot sets: leapquant_amd/_build/liblq_probe.so reads, per (row, value head) block of 64 KiB, the checkpoint bytes
    the step reads (codes, scales, factors: the first 17408 + 4 (K + V) R bytes), two blocks per 256-thread workgroup
    as the step's workgroups take them; the same bytes contiguous; and whole 64 KiB blocks -- each with plain and with
    non-temporal 16-byte loads, in graphs of 64 launches (set i % NSET).  Also the fixed cost of a launch in a graph (one
    empty workgroup)."""
    blk = ssm.stride(1) * 4                                       # bytes per (slot, head) block
    nblk = B * HV
    ck = 128 * 128 + 4 * (128 + 128) + 2 * R * (128 + 128)       # codes, Sk | Sv, UQ: 19456 bytes at R = 4
    sink = torch.empty(nblk * 256, dtype=torch.int32, device=dev)
    base = [ssm.data_ptr() + (1 + B * k) * HV * blk for k in range(NSET)]

    def run(stride, nbytes, nb, nt):
        return probe_read_us(torch, stream, capture, base, stride, nbytes, nb, 2, nt, sink)

    out = {"workload": "pure streaming reads over config 1's rotated slot sets (%d sets): per (row, value head) "
                       "block of %d bytes, two blocks per 256-thread workgroup" % (NSET, blk)}
    for name, stride, nbytes in (("checkpoint", blk, ck), ("contiguous", ck, ck), ("full_block", blk, blk)):
        nbytes_launch = nblk * nbytes
        for nt, tag in ((1, "nt"), (0, "plain")):
            us = run(stride, nbytes, nblk, nt)
            out["%s_%s_us" % (name, tag)] = round(us, 3)
            out["%s_%s_gbps" % (name, tag)] = round(nbytes_launch / (us * 1e-6) / 1e9, 1)
        out["%s_bytes_per_launch" % name] = nbytes_launch
    out["empty_launch_us"] = round(run(blk, 16, 0, 0), 3)
    out["note"] = ("checkpoint = the step's read of the cache (%d of every %d bytes); contiguous = the same bytes "
                   "without gaps; full_block = every byte of the fp32 cache" % (ck, blk))
    return out


def dense_rmw_ceiling(torch, stream, Sd, B, HV, NSET, capture):
    """The ceiling of the bf16-state baseline's access pattern: liblq_probe.so reads each (row, value head) block of the
    dense bf16 state (32 KiB) and writes it back in place (unchanged), two blocks per 256-thread workgroup as the
    baseline's workgroups take them, over the same rotated sets, in graphs of 64 launches; plain and non-temporal."""
    import ctypes
    probe = ctypes.CDLL(os.path.join(ROOT, "leapquant_amd", "_build", "liblq_probe.so"))
    probe.lq_probe_rmw.restype = ctypes.c_int
    probe.lq_probe_rmw.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_uint, ctypes.c_void_p]
    blk = Sd.stride(1) * Sd.element_size()
    nblk = B * HV
    base = [Sd.data_ptr() + (1 + B * k) * HV * blk for k in range(NSET)]
    out = {"workload": "read and write back each %d-byte (row, value head) block of the dense bf16 state, two per "
                       "256-thread workgroup, %d rotated sets" % (blk, NSET)}
    for nt, tag in ((0, "plain"), (1, "nt")):
        def launch(i, nt=nt):
            rc = probe.lq_probe_rmw(ctypes.c_void_p(base[i % NSET]), blk, blk, nblk, 2, nt, 0,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if rc:
                raise RuntimeError("lq_probe_rmw failed (%d)" % rc)
        gr = capture(launch, 64)
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()                                  # warm-up replays (default stream) done
        with torch.cuda.stream(stream):
            torch.cuda._sleep(2_000_000)                # keeps the GPU busy while the host enqueues
            e0.record(stream)
            for _ in range(4):
                gr.replay()
            e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (64 * 4)
        out["%s_us" % tag] = round(us, 3)
        out["%s_gbps" % tag] = round(2 * nblk * blk / (us * 1e-6) / 1e9, 1)
        del gr
    out["bytes_per_launch"] = 2 * nblk * blk
    return out


def traffic_bytes(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this command, each
    scaled by what the counter reads for the 64 MiB copies the bench ends with (None when the summary is absent)."""
    p = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get(kernel, {}).get("hbm_bytes_per_launch")


def _cpu_worker(heads, seed, calls, barrier, out):
    """One host process of the CPU baseline: `calls` decode calls (step + flush) of config 0 on its own `heads` value
    heads (GQA 1: each with its own key head), timed between a barrier shared by all workers and its last call."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import lq_oracle as O
    from tests.fixtures import gate_params, make_inputs, make_state
    with threadpool_limits(limits=1):
        rng = np.random.default_rng(seed)
        st, S, Q0 = make_state(rng, 2, heads, heads, L=64)
        A_log, dt_bias = gate_params(heads)
        idx = np.array([1])
        pool = [make_inputs(rng, 1, heads, heads) for _ in range(8)]
        barrier.wait()
        t0 = time.perf_counter()
        for n in range(calls):
            mixed, a, b = pool[n % 8]
            O.gdn_step(st, mixed, a, b, A_log, dt_bias, idx)
            O.flush(st, Q0, idx)
        out.put((t0, time.perf_counter()))


def cpu_baseline(target_seconds=10.0):
    """The CPU oracle (numpy) on config 0: GDN B = 1, HV = H = 16, d = 128, W = 64, R = 4, decode calls of step + flush,
    on the host's cores: the 16 heads are independent (GQA 1), so they are split over one process per core (at most
    16, the box's share, and one per head).  Runs before anything touches the GPU (the workers are forked).  The call
    count is a multiple of 256 (four windows: every head flushes once per 64 calls) sized to ~target_seconds of wall
    time from a one-process calibration.  Returns the wall time per decode call of the whole batch."""
    import multiprocessing as mp
    import numpy as np
    from oracle import lq_oracle as O
    from tests.fixtures import gate_params, make_inputs, make_state
    HV = 16
    try:
        ncpu = len(os.sched_getaffinity(0))
    except AttributeError:
        ncpu = os.cpu_count() or 1
    P = max(1, min(ncpu, 16, HV))
    split = [HV // P + (1 if i < HV % P else 0) for i in range(P)]
    # calibration: 64 calls of the largest worker's share, one process
    rng = np.random.default_rng(999)
    st, S, Q0 = make_state(rng, 2, max(split), max(split), L=64)
    A_log, dt_bias = gate_params(max(split))
    mixed, a, b = make_inputs(rng, 1, max(split), max(split))
    t0 = time.perf_counter()
    for _ in range(64):
        O.gdn_step(st, mixed, a, b, A_log, dt_bias, np.array([1]))
        O.flush(st, Q0, np.array([1]))
    per_call = (time.perf_counter() - t0) / 64
    calls = 256 * max(1, min(64, int(target_seconds / (256 * per_call))))
    ctx = mp.get_context("fork")
    barrier = ctx.Barrier(P)
    out = ctx.Queue()
    procs = [ctx.Process(target=_cpu_worker, args=(split[i], 1000 + i, calls, barrier, out)) for i in range(P)]
    for p in procs:
        p.start()
    spans = [out.get() for _ in procs]
    for p in procs:
        p.join()
    if any(p.exitcode != 0 for p in procs):
        raise RuntimeError("a CPU baseline worker failed")
    wall = max(t1 for _, t1 in spans) - min(t0 for t0, _ in spans)
    us = wall / calls * 1e6
    nbytes = (sum(step_bytes(1, HV, HV, 128, 128, 4, h) for h in range(64)) / 64
              + flush_bytes(1, HV, HV, 128, 128, 4, 64) / 64)
    return dict(value=round(us, 1), unit="us/step", cores=P, kind="port",
                gbps=round(nbytes / (us * 1e-6) / 1e9, 3), host_cpus=ncpu,
                sample="config 0 (GDN B=1, HV=H=16, d=128, W=64, R=4): %d decode calls (step + flush, %d flushes) of "
                       "the numpy oracle, its 16 independent heads split over %d host processes (%s heads each), one "
                       "BLAS thread per process; wall time per call" % (calls, calls // 64, P,
                                                                       "/".join(str(x) for x in sorted(set(split)))))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--sets", type=int, default=8, help="disjoint slot sets rotated through (MALL defeat)")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the decode path shards heads across "
              "GPUs with no exchange step; see the design notes)", file=sys.stderr)
        sys.exit(2)
    if 64 % args.sets:
        print("--sets must divide 64 (each graph of 64 launches gives every set the same number of steps)",
              file=sys.stderr)
        sys.exit(2)
    cpu = None
    if not args.no_cpu:                        # host processes are forked before anything touches the GPU
        cpu = cpu_baseline()
        progress("CPU baseline: %.1f us per call on %d processes" % (cpu["value"], cpu["cores"]))

    import torch
    from leapquant_amd import kernels as KN
    from leapquant_amd.state import LeapQuantState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, HV, H, K, V, L, R = 64, 32, 16, 128, 128, 64, 4
    NSET = args.sets
    NS = B * NSET + 1
    g = torch.Generator(device=dev)
    g.manual_seed(1001)

    # ---- state: N(0, 0.02^2) fp32 per head, quantised on the GPU ----
    ssm = torch.empty(NS, HV, V, K, device=dev)
    ssm.normal_(0.0, 0.02, generator=g)
    lq = LeapQuantState(ssm, H, L=L, R=R)
    all_slots = torch.arange(1, NS, device=dev, dtype=torch.int32)
    lq.quantize(ssm, all_slots)
    sets = [torch.arange(1 + B * k, 1 + B * (k + 1), device=dev, dtype=torch.int32) for k in range(NSET)]

    # ---- input pool (config-0 distributions), resident in HBM ----
    P = 16
    pool = []
    for _ in range(P):
        q = torch.randn(B, H, K, device=dev, generator=g)
        k = torch.randn(B, H, K, device=dev, generator=g)
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(B, HV, V, device=dev, generator=g)
        mixed = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], 1).to(torch.bfloat16).contiguous()
        gl = -0.1 * torch.rand(B, HV, device=dev, generator=g)
        gl = gl.clamp(max=-1e-4)
        a = torch.log(torch.expm1(-gl)).to(torch.bfloat16)
        b = torch.randn(B, HV, device=dev, generator=g).to(torch.bfloat16)
        pool.append((mixed, a, b))
    A_log = torch.zeros(HV, device=dev)
    dt_bias = torch.zeros(HV, device=dev)
    out = torch.empty(B, HV, V, device=dev, dtype=torch.bfloat16)

    def decode(s):
        mixed, a, b = pool[s % P]
        lq.decode(ssm, mixed, a, b, A_log, dt_bias, sets[s % NSET], out)

    def reset_windows(q):
        """Every window of state q back to empty (h = 0; weights 0, decay product 1), the checkpoints kept: the timed
        loops after the first start from there, as after a flush."""
        q.hcnt.zero_()
        q.Wbuf.zero_()
        q.Pbuf.fill_(1.0)

    v = lq.views(ssm)

    def step_only(s, kset):
        mixed, a, b = pool[s % P]
        lq.kstep(v["q32"], v["Sk"], v["Sv"], v["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.hcnt, mixed, a, b,
                 A_log, dt_bias, v["uq"], sets[kset], out)

    def flush_only(kset):
        lq.kflush(v["q32"], v["Sk"], v["Sv"], v["skv"], lq.Kbuf, lq.Ubuf, lq.Wbuf, lq.Pbuf, lq.Gd, lq.hcnt,
                  v["sq16"], v["uq"], lq.Q0, sets[kset])

    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    def capture(fn, n):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            for i in range(n):
                fn(i)
        return gr

    # ---- main loop: decode (step + flush) in graphs of 64 calls ----
    # The graph's call i uses set i % NSET and input i % P.  A rotation is NSET replays (L * NSET calls): every set's
    # windows go from empty through the full-window flush back to empty, so a timed region of whole rotations holds
    # each window fill h = 0..63 and each flush in its real proportion, whatever --steps is (rounded up to rotations).
    CH = 64
    ROT = L * NSET
    gdec = capture(decode, CH)
    torch.cuda.synchronize()                                      # capturing executes nothing
    # at least two rotations of warm-up: under continuous load the second rotation still ran ~1% slower than the third
    # and later ones (16.61 against 16.45 us per call)
    warm_rot = max(2, -(-args.warmup // ROT))
    timed_rot = max(1, -(-args.steps // ROT))
    tev = [torch.cuda.Event(enable_timing=True) for _ in range(timed_rot + 1)]   # between rotations: no gap added
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        # the warm-up replays are queued right before the timed ones, so the GPU goes from them into the timed region
        # without idling (after an idle gap of ~1 ms the first timed rotation ran 2-3% slower: 16.83 against 16.45 us per
        # call) and they keep it busy while the host enqueues the timed replays
        for _ in range(warm_rot * NSET):
            gdec.replay()
        tev[0].record(stream)
        for k in range(timed_rot):
            for _ in range(NSET):
                gdec.replay()
            tev[k + 1].record(stream)
    tev[-1].synchronize()
    torch.cuda.synchronize()
    assert int(lq.hcnt[1:].max()) == 0                           # whole rotations: every window back at its start
    ms_total = tev[0].elapsed_time(tev[-1])
    calls = timed_rot * ROT
    us_per_step = ms_total * 1e3 / calls
    timed_rot_us = [round(tev[k].elapsed_time(tev[k + 1]) * 1e3 / ROT, 3) for k in range(timed_rot)]
    # bytes of exactly those calls: per set and window, the 64 steps at fills 0..63 and one all-due flush
    timed_bytes = timed_rot * NSET * (sum(step_bytes(B, HV, H, K, V, R, h) for h in range(L))
                                      + flush_bytes(B, HV, H, K, V, R, L))

    decode_gbps = timed_bytes / (ms_total * 1e-3) / 1e9
    progress("decode loop: %.3f us per call over %d calls (%d whole rotations of %d sets; per rotation %s)"
             % (us_per_step, calls, timed_rot, NSET, timed_rot_us))
    # spread of the same figure: µs per call of each of SPREAD_ROT further whole rotations, events between them (no
    # gap in the GPU's work), after an untimed rotation queued right before them as above; the windows are back at
    # their start after every rotation
    SPREAD_ROT = 9
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(SPREAD_ROT + 1)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(NSET):
            gdec.replay()
        evs[0].record(stream)
        for k in range(SPREAD_ROT):
            for _ in range(NSET):
                gdec.replay()
            evs[k + 1].record(stream)
    torch.cuda.synchronize()
    import numpy as np
    rot_us = np.array([evs[k].elapsed_time(evs[k + 1]) * 1e3 / ROT for k in range(SPREAD_ROT)])
    value_spread = {"rotations": SPREAD_ROT, "calls_each": ROT, "median": round(float(np.median(rot_us)), 3),
                    "p10": round(float(np.percentile(rot_us, 10)), 3), "p90": round(float(np.percentile(rot_us, 90)), 3),
                    "min": round(float(rot_us.min()), 3), "max": round(float(rot_us.max()), 3)}
    # ---- staggered windows (beside the BASELINE workload, not it): row n of every set starts at fill n % 64, so on
    # every call one row per set fills its window and is flushed, as in serving, where rows reach their flush at
    # different calls; the same decode graph over whole rotations ----
    fill0 = (torch.arange(B, device=dev, dtype=torch.int32) % L)[:, None].expand(B, HV)
    for kk in range(NSET):
        lq.hcnt[sets[kk].long()] = fill0
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(2 * NSET):                   # warm-up queued directly before the timed replays
            gdec.replay()
        s0.record(stream)
        for _ in range(NSET):
            gdec.replay()
        s1.record(stream)
    s1.synchronize()
    staggered_us = s0.elapsed_time(s1) * 1e3 / ROT
    # the same with the step and the flush as two launches (lq_gdn_step, then lq_flush of the call's rows: every due
    # head its own workgroup), for comparison
    reset_windows(lq)
    for kk in range(NSET):
        lq.hcnt[sets[kk].long()] = fill0

    def step_then_flush(i):
        step_only(i, i % NSET)
        flush_only(i % NSET)
    gsf = capture(step_then_flush, CH)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(2 * NSET):                   # warm-up queued directly before the timed replays
            gsf.replay()
        s0.record(stream)
        for _ in range(NSET):
            gsf.replay()
        s1.record(stream)
    s1.synchronize()
    staggered_two_us = s0.elapsed_time(s1) * 1e3 / ROT
    del gsf
    # the deferred-flush decode (lq_gdn_decode_deferred: of the two heads of a key head a call fills, the second is
    # flushed at the start of the next call that steps the slot): synchronized windows, then staggered ones
    lqd = LeapQuantState(ssm, H, L=L, R=R, defer_flush=True)

    def decode_deferred(s):
        mixed, a, b = pool[s % P]
        lqd.decode(ssm, mixed, a, b, A_log, dt_bias, sets[s % NSET], out)
    gdd = capture(decode_deferred, CH)
    deferred_us = {}
    for regime in ("synchronized", "staggered"):
        reset_windows(lqd)
        if regime == "staggered":
            for kk in range(NSET):
                lqd.hcnt[sets[kk].long()] = fill0
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(2 * NSET):                   # warm-up queued directly before the timed replays
                gdd.replay()
            s0.record(stream)
            for _ in range(NSET):
                gdd.replay()
            s1.record(stream)
        s1.synchronize()
        deferred_us[regime] = s0.elapsed_time(s1) * 1e3 / ROT
    del gdd
    lqd.flush(ssm, all_slots)                                     # settle the deferred heads
    torch.cuda.synchronize()
    del lqd
    progress("decode loop, staggered windows: %.3f us per call (step + flush launches: %.3f)"
             % (staggered_us, staggered_two_us))
    # ---- step-only and flush timings, sets rotated as in the decode loop (a graph of 64 step launches gives each
    # of the NSET sets 64 / NSET steps; NSET replays take every window from h = 0 to h = 64, then every head is due) ----
    reset_windows(lq)                                             # every window back to h = 0
    gsteps = capture(lambda i: step_only(i, i % NSET), CH)
    gflush = [capture(lambda i, kk=kk: flush_only(kk), 1) for kk in range(NSET)]
    def idle_flush(i):                 # lq_flush through the layer's flagged lq_state, as a two-launch decode runs it
        import ctypes
        from leapquant_amd import _lib, kernels as KN
        st_ = lq._struct(ssm)
        _lib.check(_lib.lib().lq_flush(ctypes.byref(st_), KN._p(lq.Q0), KN._p(sets[0]), B, 0,
                                       ctypes.c_float(lq.qmax),
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "lq_flush")

    gidle = capture(idle_flush, CH)                               # 64 flush launches with no head due
    torch.cuda.synchronize()
    rounds = 3
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(NSET + 2)] for _ in range(rounds)]
    torch.cuda.synchronize()                                  # warm-up replays (default stream) done
    with torch.cuda.stream(stream):
        for r in range(rounds):
            if r == 0:
                torch.cuda._sleep(2_000_000)
            ev[r][0].record(stream)
            for _ in range(NSET):
                gsteps.replay()
            ev[r][1].record(stream)
            for kk in range(NSET):
                gflush[kk].replay()
                ev[r][kk + 2].record(stream)
        i0, i1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)                # keeps the GPU busy while the host enqueues
        i0.record(stream)
        gidle.replay()
        i1.record(stream)
    torch.cuda.synchronize()
    st_ms = [ev[r][0].elapsed_time(ev[r][1]) for r in range(1, rounds)]
    fl_ms = [ev[r][kk + 1].elapsed_time(ev[r][kk + 2]) for r in range(1, rounds) for kk in range(NSET)]
    step_us = sum(st_ms) / len(st_ms) * 1e3 / (CH * NSET)
    flush_due_us = sum(fl_ms) / len(fl_ms) * 1e3
    flush_idle_us = i0.elapsed_time(i1) * 1e3 / CH
    bytes_step = sum(step_bytes(B, HV, H, K, V, R, h) for h in range(CH)) / CH      # mean over h = 0..63
    bytes_flush = flush_bytes(B, HV, H, K, V, R, L)
    achieved = bytes_step / (step_us * 1e-6) / 1e9

    progress("step %.3f us, flush due %.1f us, idle %.2f us" % (step_us, flush_due_us, flush_idle_us))
    # ---- bf16-state baseline (same step on a dense bf16 state), rotated sets ----
    del gsteps, gflush, gidle, gdec
    Sd = torch.empty(NS, HV, V, K, device=dev, dtype=torch.bfloat16)
    Sd.normal_(0.0, 0.02, generator=g)

    def dense(i):
        mixed, a, b = pool[i % P]
        KN.dense_step(Sd, mixed, a, b, A_log, dt_bias, sets[i % NSET], out, H)

    gd = capture(dense, CH)
    d0, d1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(2 * NSET):                   # warm-up queued directly before the timed replays, as for the decode
            gd.replay()
        d0.record(stream)
        for _ in range(2 * NSET):
            gd.replay()
        d1.record(stream)
    torch.cuda.synchronize()
    bf16_us = d0.elapsed_time(d1) * 1e3 / (2 * NSET * CH)
    bf16_gbps = dense_bytes(B, HV, H, K, V) / (bf16_us * 1e-6) / 1e9
    rmw = dense_rmw_ceiling(torch, stream, Sd, B, HV, NSET, capture)
    del gd, Sd

    # ---- conv1d update fused into the step (lq_gdn_step_conv) against the conv update kernel + step, same rotated
    # sets and raw projections (the pool's mixed rows stand for the raw in_proj output); windows from h = 0 ----
    import ctypes
    from leapquant_amd import _lib
    C = 2 * H * K + HV * V
    conv = torch.empty(NS, C, 3, device=dev).normal_(0.0, 1.0, generator=g).to(torch.bfloat16)
    cw = (torch.empty(C, 4, device=dev).normal_(0.0, 0.5, generator=g)).to(torch.bfloat16).contiguous()
    cv = KN.conv_struct(conv, cw, None, True)
    xconv = torch.empty(B, C, device=dev, dtype=torch.bfloat16)
    sts = lq._struct(ssm)
    ios = {}

    def io_of(x, a, b, kset):
        key = (x.data_ptr(), a.data_ptr(), kset)
        if key not in ios:
            ios[key] = KN._step_io(x, a, b, A_log, dt_bias, sets[kset], out, K ** -0.5)
        return ios[key]

    def fused(i):
        x, a, b = pool[i % P]
        _lib.check(_lib.lib().lq_gdn_step_conv(ctypes.byref(sts), ctypes.byref(io_of(x, a, b, i % NSET)),
                                                ctypes.byref(cv), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "lq_gdn_step_conv")

    def unfused(i):
        x, a, b = pool[i % P]
        KN.conv_update(x, conv, cw, None, sets[i % NSET], xconv, True)
        _lib.check(_lib.lib().lq_gdn_step(ctypes.byref(sts), ctypes.byref(io_of(xconv, a, b, i % NSET)),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "lq_gdn_step")

    def fused_decode(i):                                          # what the plugin runs for a bf16 conv of width 4
        x, a, b = pool[i % P]
        lq.decode_conv(ssm, x, conv, cw, None, True, a, b, A_log, dt_bias, sets[i % NSET], out)

    conv_us = {}
    for name, fn in (("fused", fused), ("unfused", unfused), ("decode", fused_decode)):
        gr = capture(fn, CH)
        reset_windows(lq)                                         # every window back to h = 0
        torch.cuda.synchronize()
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()                                  # warm-up replays (default stream) done
        with torch.cuda.stream(stream):
            torch.cuda._sleep(2_000_000)                # keeps the GPU busy while the host enqueues
            c0.record(stream)
            for _ in range(NSET):                                 # every set steps h = 0 .. 63
                gr.replay()
            c1.record(stream)
        torch.cuda.synchronize()
        conv_us[name] = c0.elapsed_time(c1) * 1e3 / (NSET * CH)
        del gr
    del conv, xconv

    # ---- 8 copies of 64 MiB: the known-size kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters when this
    # same command runs under rocprofv3 --pmc (bytes per launch of the step: profiles/hbm_traffic.json) ----
    src = torch.empty(64 * 2 ** 20 // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst

    progress("bf16 baseline, fused conv, calibration copies")
    ceiling = loader_ceiling(torch, dev, stream, ssm, B, HV, NSET, R, capture)
    progress("loader ceiling")
    kda = kda_bench(torch, dev, stream, capture)
    progress("KDA config 2")
    fq = flush_quantize_bench(torch, dev, stream)
    progress("config-3 flush / quantize")
    hd = head_dims_bench(torch, dev, stream, capture)
    progress("head-dim variants")

    res = {
        "metric": METRIC, "value": round(us_per_step, 3), "unit": "us/step", "n_gpus": 1, "steps": calls,
        "warmup": warm_rot * ROT, "steps_requested": args.steps, "warmup_requested": args.warmup,
        "steps_note": "decode calls timed: --steps rounded up to whole rotations of %d calls (every set's window "
                      "from empty through its flush), so flushes are timed in their real proportion; warm-up: "
                      "--warmup rounded up to whole rotations, at least 2, queued directly before the timed calls" % ROT,
        "ms_per_step": round(us_per_step / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "GDN decode, BASELINE config 1: B=64, HV=32 value / H=16 key heads, d=128, W=64, R=4, "
                               "int8 state + fp32 scales, step + flush per call (the flush does work on one call in "
                               "64), whole windows of %d rotated slot sets" % NSET,
                   "batch": B, "value_heads": HV, "key_heads": H, "head_dim": K, "window": L, "rank": R},
        "achieved_gbps": round(decode_gbps, 1),
        "value_spread": value_spread,
        "bf16_state_step_us": round(bf16_us, 3), "bf16_state_gbps": round(bf16_gbps, 1),
        "bf16_state_rmw_ceiling": rmw,
        "speedup_vs_bf16_step": round(bf16_us / us_per_step, 3),
        # the timed region is one kernel per decode call: the step that flushes the heads it fills
        "roofline": {"bound": "hbm", "achieved": round(decode_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(decode_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic_bytes(DECODE_KERNEL),
                     "kernel": DECODE_KERNEL, "bytes_per_launch": int(timed_bytes / calls),
                     "us_per_launch": round(us_per_step, 3)},
        # the step alone (no flush work), every window fill h = 0..63 over the same rotated sets
        "step_us": round(step_us, 3), "speedup_vs_bf16_step_alone": round(bf16_us / step_us, 3),
        "step_roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic_bytes(STEP_KERNEL),
                          "kernel": STEP_KERNEL, "bytes_per_launch": int(bytes_step)},
        # the standalone flush kernel (lq_flush: the KDA path, the other head shapes, the reference-API factories)
        "flush_due_us": round(flush_due_us, 2), "flush_idle_us": round(flush_idle_us, 3),
        "decode_staggered_us": round(staggered_us, 3),
        "decode_staggered_two_launch_us": round(staggered_two_us, 3),
        "decode_deferred_us": round(deferred_us["synchronized"], 3),
        "decode_staggered_deferred_us": round(deferred_us["staggered"], 3),
        "decode_staggered_note": "not the BASELINE workload: row n starts at window fill n % 64, so on every call one "
                                 "row per set is flushed (rows reach their flush at different calls, as in serving); "
                                 "deferred = lq_gdn_decode_deferred (LeapQuantState(defer_flush=True)): of the two "
                                 "heads of a key head a call fills, the second is flushed at the start of the next "
                                 "call that steps the slot (same outputs)",
    }
    res["conv_fused_config1"] = {
        "workload": "config 1 step with vLLM's causal_conv1d_update (width 4, SiLU, bf16 state [NS, C, 3]) fused in, "
                    "against the conv update kernel + step; rotated sets, h = 0..63",
        "fused_step_us": round(conv_us["fused"], 3), "conv_then_step_us": round(conv_us["unfused"], 3),
        "plain_step_us": round(step_us, 3),
        "decode_conv_us": round(conv_us["decode"], 3),
        "decode_conv_note": "LeapQuantState.decode_conv (lq_gdn_decode with the conv): conv + step + the flushes of "
                            "the heads it fills, one launch per call, one whole window of every set"}
    res["loader_ceiling"] = ceiling
    res["kda_config2"] = kda
    res["flush_quantize_config3"] = fq
    res["head_dims_W16"] = hd
    if cpu is not None:
        res["cpu_baseline"] = cpu
    print(json.dumps(res))


if __name__ == "__main__":
    main()
