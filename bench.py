"""Throughput of the Qwen3-TTS frame step on one MI355X.

A step is one frame step (TQwenTalker.NextFrame, src/tts/mormot.ai.tts.qwen.
talker.pas:640-681): for every stream, code 0 from the talker logits, 15
code-predictor forwards (5 layers) each with its head and argmax, the sum of
16 embeddings, one talker forward (28 layers) with the 3072-code head, and
the 16 codes of each stream copied back to the host.

Workloads (random-init N(0, 0.02) weights from a seed, Q8_0, norm weights 1,
synthetic N(0, 1) prompt embeddings; nothing is downloaded):
  frame_b1   1 stream, 48 prompt rows, K frames (156: context 48 -> 204)
  frame_b32  32 streams, prompt rows uniform in [16, 256] (seeded), K frames;
             activations quantized per 32-block (int8 MFMA products)

Timed region: K steps after W warm-up steps; the warm-up runs on a first
prefill, the timed steps restart from a fresh prefill so that the context
grows exactly as in the workload. Each step returns with its codes in host
memory, so the wall clock of the K calls is the whole-job time.

Beside it:
  roofline      the Q8_0 matrix-vector products of one talker decode step (28
                layers x 4 products + the 3072-row head, 471.5 MB of weights,
                more than the 256 MB Infinity Cache holds): the average launch
                duration of the products captured in a HIP graph and replayed
                between two HIP events on their stream (gaps included), with
                direct launches and an event pair on each launch beside it,
                the rocprofv3 trace's average of the same products, and the
                bound one dependent launch of that many bytes can reach;
  cpu_baseline  the oracle (the C restatement of the same frame step) on the
                host cores, on a bounded sample of the same workload;
  batched_b32 (frame_b1)  32 streams, prompt rows uniform in [16, 256],
                128 frames, int8 activations (int8 MFMA products);
  f32_b8 (frame_b1)  f32 weights at batch 8: 8 x 512-row prefills, then 64
                frames of f32 products, with the oracle's f32 frame step as
                its CPU baseline and stream 0's codes against it;
  decode_attention_b1 (frame_b1)  the frame's talker decode attention at
                batch 1 (f32 K/V) at 64, 126, 192 and 256 positions: us per
                layer and GB/s;
  long_context_attention (frame_b1)  the talker with an f16 K/V cache
                prefilled to 2048 / 4096 / 8192 positions: 32 decode steps
                each, and the decode attention kernels' GB/s;
  codec_back (frame_b1)  the 12 Hz decoder's back part (2.46 GMAC per frame)
                over 156 frames: passes of 16 frames and one frame per call;
  start_from_text (frame_b1)  time to the first frame from token ids: the
                text projection, the prefill rows built on the device, the
                talker prefill and one frame step (a 40-token sentence).

Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mormot2-qwen-tts_amd")
sys.path.insert(0, PKG)

import q3h  # noqa: E402
import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
F32_MFMA_PEAK_TFLOPS = 157.3
F32_PROMPT_ROWS = 512
# HBM bytes per launch of the single-row Q8_0 products of one talker decode
# step, from rocprofv3 FETCH_SIZE + WRITE_SIZE passes scaled by a plain copy
# kernel of known size (profiles/gemv_q8_decode_step_traffic.md)
GEMV_TRAFFIC_PER_LAUNCH = 4320854
# the same products' average duration in a rocprofv3 kernel trace (5,876
# direct dispatches; profiles/gemv_q8_decode_step_durations.md)
GEMV_ROCPROF_US_PER_LAUNCH = 3.273
# what one dependent launch of a product can reach on this part: an empty
# kernel costs LAUNCH_FLOOR_US per dependent launch in a graph before any byte
# moves, and HBM streams HBM_MARGINAL_GBS marginal (4 MB / 8 MB launches)
LAUNCH_FLOOR_US = 1.54
HBM_MARGINAL_GBS = 5700.0
PROMPT_ROWS = 48


def log(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def build_model(dev, seed, max_positions, act_q8, dtype=q3h.Q8_0, kv16=0):
    """Talker + code predictor + heads on the device, from f32 weights that the
    library quantizes to Q8_0 (bit-exact ggml quantize_row_q8_0_ref) or keeps
    in f32 (dtype F32); act_q8: activations quantized per 32-block too (int8
    MFMA products)."""
    t0 = time.time()
    tl, tf = synth.stack_weights(seed, "talker.model.", synth.TALKER)
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=dtype, kv_f16=kv16, act_q8=act_q8,
                             max_positions=max_positions), tl, tf, q3h.F32)
    cl, cf = synth.stack_weights(seed, "talker.code_predictor.model.", synth.PREDICTOR)
    cs = q3h.Stack(dev, dict(synth.PREDICTOR, dtype=dtype, kv_f16=kv16, act_q8=act_q8,
                             max_positions=16), cl, cf, q3h.F32)
    th = synth.talker_head(seed)
    ts.add_head(th, q3h.F32)
    ch = [synth.cp_head(seed, g) for g in range(15)]
    for h in ch:
        cs.add_head(h, q3h.F32)
    tables = dict(codec_emb=synth.codec_embedding(seed),
                  pred_emb=[synth.pred_embedding(seed, g) for g in range(15)],
                  tts_pad=synth.tts_pad(seed))
    log(f"model on the device in {time.time() - t0:.1f} s "
        f"({(ts.bytes + cs.bytes) / 1e6:.1f} MB of layers)")
    f32 = dict(tl=tl, tf=tf, cl=cl, cf=cf, th=th, ch=ch)
    return ts, cs, tables, f32


def load_from_bf16(dev, f32, act_q8, dtype=q3h.Q8_0):
    """The load path of the reference (safetensors BF16 rows -> device weights,
    lm.pas:244-308): both stacks and their 16 heads created from BF16 host
    rows, widened and quantized on the device. Seconds of the creation calls
    (the host BF16 rows prepared beforehand, untimed)."""
    b = synth.to_bf16_bits

    def rows(layers):
        return [{k: (b(v) if k.startswith("w") else v) for k, v in L.items()} for L in layers]
    tl, cl = rows(f32["tl"]), rows(f32["cl"])
    th, ch = b(f32["th"]), [b(h) for h in f32["ch"]]
    nbytes = sum(v.nbytes for L in tl + cl for k, v in L.items() if k.startswith("w"))
    nbytes += th.nbytes + sum(h.nbytes for h in ch)
    t0 = time.perf_counter()
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=dtype, kv_f16=0, act_q8=act_q8,
                             max_positions=64), tl, f32["tf"], q3h.BF16)
    cs = q3h.Stack(dev, dict(synth.PREDICTOR, dtype=dtype, kv_f16=0, act_q8=act_q8,
                             max_positions=16), cl, f32["cf"], q3h.BF16)
    ts.add_head(th, q3h.BF16)
    for h in ch:
        cs.add_head(h, q3h.BF16)
    dt = time.perf_counter() - t0
    ts.destroy()
    cs.destroy()
    log(f"load from BF16 rows: {dt:.2f} s ({nbytes / 1e9:.2f} GB of BF16 weights)")
    return dict(seconds=round(dt, 3), bf16_bytes=int(nbytes),
                what="talker (28 layers) + code predictor (5 layers) + 16 heads, BF16 host rows "
                     "-> Q8_0 on the device")


def prompts(seed, workload, n, rows=PROMPT_ROWS):
    if workload == "frame_b1":
        return [synth.prompt(seed, rows)]
    if workload == "f32_b8":
        return [synth.prompt(seed + 2000 + s, F32_PROMPT_ROWS) for s in range(n)]
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = rng.integers(16, 257, size=n)
    return [synth.prompt(seed + 1000 + s, int(L)) for s, L in enumerate(lens)]


def start_all(frame, pre):
    """Start every stream: one stream with q3h_frame_start, several with
    q3h_frame_start_batch (their prefills overlapping on the device)."""
    if len(pre) == 1:
        frame.start(0, pre[0])
    else:
        frame.start_batch(list(range(len(pre))), pre)


def start_one_by_one(frame, pre):
    """Seconds of one q3h_frame_start per stream, each waited for (the
    reference's way: one sentence at a time)."""
    t0 = time.perf_counter()
    for s, p in enumerate(pre):
        frame.start(s, p)
    return time.perf_counter() - t0


def run_gpu(frame, pre, steps, warmup):
    start_all(frame, pre)
    for _ in range(warmup):
        frame.step()
    t0 = time.perf_counter()
    start_all(frame, pre)
    run_gpu.prefill_s = time.perf_counter() - t0
    lat = np.empty(steps)
    codes = []
    t0 = time.perf_counter()
    for i in range(steps):
        a = time.perf_counter()
        c, alive = frame.step()
        lat[i] = time.perf_counter() - a
        codes.append(c)
    total = time.perf_counter() - t0
    return total, lat, np.stack(codes)


def cpu_info():
    """The host CPU as /proc/cpuinfo names it, and the vector ISA the oracle
    is built for (-march=x86-64-v3: AVX2, FMA, F16C) with the wider
    extensions the CPU also has."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    extra = [x for x in ("avx512f", "avx512_vnni", "avx512_bf16", "amx_tile") if x in flags]
    return dict(cpu_model=model, isa="x86-64-v3 (AVX2, FMA, F16C) build" +
                (f"; the CPU also has {', '.join(extra)}" if extra else ""))


def cpu_thread_counts():
    """The host cores this job may use (at most 16: one GPU's share of an
    8-GPU host) and the reference's default worker count for them,
    (2 nproc + 2) / 3 (mormot.ai.tts.qwen.talker.pas:316-317)."""
    share = min(16, len(os.sched_getaffinity(0)))
    return sorted({max(1, (2 * share + 2) // 3), share})


def cpu_baseline(f32, tables, pre, gpu_codes, budget_s, max_frames, act_q8, f32w=False):
    """The oracle's frame step on the host cores (same weights, same prompt of
    stream 0, same weight and activation modes), frames timed until budget_s
    is spent, at each of cpu_thread_counts(); value: the faster."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import q3o  # the oracle, timed as the CPU baseline

    q3o.set_threads(max(cpu_thread_counts()))
    ot, oc, frame = oracle_model(q3o, f32, tables, act_q8, f32w,
                                 pre[0].shape[0] + max_frames + 8)
    sweep = [cpu_frames(q3o, frame, pre, gpu_codes, budget_s, max_frames, threads)
             for threads in cpu_thread_counts()]
    ot.destroy()
    oc.destroy()
    best = max(sweep, key=lambda r: r["value"])
    n = max(r["frames"] for r in sweep)
    equal = all(r["codes_equal"] for r in sweep)
    act = "int8 activations" if act_q8 else "f32 activations"
    wts = "f32 weights" if f32w else "Q8_0 weights"
    out = dict(value=round(best["value"], 3), unit="frames/s", cores=best["threads"],
               kind="port",
               sample=f"frame step of stream 0, {wts}, {act} (oracle, C + OpenMP), "
                      f"{pre[0].shape[0]} prompt rows (prefill untimed), the first frames for "
                      f"about {budget_s:.0f} s at each thread count",
               threads_sweep=[dict(threads=r["threads"], frames_per_s=round(r["value"], 3),
                                   frames=r["frames"], seconds=round(r["seconds"], 2))
                              for r in sweep],
               thread_counts="(2 nproc + 2) / 3 (talker.pas:316-317) and nproc, nproc = "
                             "min(16, host cores available)")
    out.update(cpu_info())
    return out, n, equal


def oracle_model(q3o, f32, tables, act_q8, f32w, max_positions):
    """The oracle's stacks and a frame factory over the same weights (Q8_0
    blocks from the same quantizer as the device's, or f32)."""
    q = (lambda v: v) if f32w else q3o.quantize_q8_0

    def qlayers(layers):
        return [{k: (q(v) if k.startswith("w") else v) for k, v in L.items()} for L in layers]

    wt = q3o.F32 if f32w else q3o.Q8_0
    ot = q3o.Stack(synth.TALKER, qlayers(f32["tl"]), f32["tf"], wt, act_q8=act_q8)
    oc = q3o.Stack(synth.PREDICTOR, qlayers(f32["cl"]), f32["cf"], wt, act_q8=act_q8)
    th, ch = q(f32["th"]), [q(h) for h in f32["ch"]]

    def frame():
        return q3o.Frame(ot, oc, th, ch, tables["codec_emb"], tables["pred_emb"],
                         tables["tts_pad"], max_positions=max_positions)
    return ot, oc, frame


def cpu_frames(q3o, frame, pre, gpu_codes, budget_s, max_frames, threads):
    """Frames of stream 0 on `threads` host threads until budget_s is spent
    (at least 2), and whether their codes equal the GPU's."""
    q3o.set_threads(threads)
    fr = frame()
    fr.start(pre[0])
    n = 0
    equal = True
    t0 = time.perf_counter()
    while n < max_frames and (n < 2 or time.perf_counter() - t0 < budget_s):
        c = fr.next()
        equal = equal and n < len(gpu_codes) and np.array_equal(c, gpu_codes[n][0])
        n += 1
    dt = time.perf_counter() - t0
    fr.destroy()
    log(f"cpu baseline: {n / dt:.2f} frames/s on {threads} threads ({n} frames)")
    return dict(value=n / dt, threads=threads, frames=n, seconds=dt, codes_equal=equal)


def gemv_roofline(ts, args, cs=None):
    """The dominant kernel: the Q8_0 matrix-vector products of one talker
    decode step. achieved = algorithmic bytes per launch / the average launch
    duration: the step's products captured in a HIP graph on their own stream
    and replayed iters times between two HIP events recorded on that stream
    (mode 1 of q3h_stack_time_gemv), as the frame step runs them; the gaps
    between launches count against the kernels. Beside it: the same products
    launched directly between two events (mode 0: there the host's launch
    rate can leave the device idle between kernels) and with an event pair
    attached to each launch (mode 2: that timing adds its own cost to every
    launch). With --no-graph the direct launches give the figure. With cs:
    the same for one code-predictor forward (5 layers + one 2048-row head,
    85.8 MB: after the first pass its weights stay in the 256 MB Infinity
    Cache)."""
    direct, launches, nbytes = ts.time_gemv(head=0, iters=args.gemv_iters, mode=0)
    ev_us, _, _ = ts.time_gemv(head=0, iters=args.gemv_iters, mode=2)
    wall = None
    if not args.no_graph:
        wall, _, _ = ts.time_gemv(head=0, iters=args.gemv_iters, mode=1)
    us = direct if wall is None else wall
    per_launch = nbytes / launches
    achieved = per_launch / (us * 1e-6) / 1e9
    log(f"gemv: {launches} launches/step, {us:.2f} us/launch ({achieved:.0f} GB/s, "
        f"{'direct launches' if wall is None else 'graph replay'}), direct launches "
        f"{direct:.2f} us, events on each launch {ev_us:.2f} us")
    # the bound one launch of per_launch bytes can reach: the launch floor plus
    # the bytes at the marginal HBM rate
    attain_us = LAUNCH_FLOOR_US + per_launch / (HBM_MARGINAL_GBS * 1e3)
    attain = per_launch / (attain_us * 1e-6) / 1e9
    rp = per_launch / (GEMV_ROCPROF_US_PER_LAUNCH * 1e-6) / 1e9
    out = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
               frac=round(achieved / HBM_PEAK_GBS, 4), traffic=GEMV_TRAFFIC_PER_LAUNCH,
               frac_basis=("graph-replayed wall time per launch (gaps between launches "
                           "included)" if wall is not None else "direct launches"),
               rocprof=dict(us_per_launch=GEMV_ROCPROF_US_PER_LAUNCH, achieved=round(rp, 1),
                            frac=round(rp / HBM_PEAK_GBS, 4),
                            source="profiles/gemv_q8_decode_step_durations.md (kernel trace "
                                   "of the same products, direct launches)"),
               attainable_per_launch=dict(
                   us=round(attain_us, 3), achieved=round(attain, 1),
                   frac=round(attain / HBM_PEAK_GBS, 4),
                   frac_reached=round(achieved / attain, 4),
                   model=f"{LAUNCH_FLOOR_US} us per dependent launch (empty kernel in a graph) "
                         f"+ bytes at {HBM_MARGINAL_GBS / 1e3:.1f} TB/s marginal HBM rate"),
               traffic_source="profiles/gemv_q8_decode_step_traffic.md",
               kernel="k_gemv_q8v (Q8_0 matrix-vector products of one talker decode step)",
               bytes_per_launch=int(per_launch), us_per_launch=round(us, 3),
               timing=("direct launches between two events on their stream (gaps included)"
                       if wall is None else "graph replay between two events on its stream "
                       "(gaps included)"),
               direct_us_per_launch=round(direct, 3),
               event_attached_us_per_launch=round(ev_us, 3),
               graph_wall_us_per_launch=None if wall is None else round(wall, 3))
    if cs is not None:
        cdirect, cl, cb = cs.time_gemv(head=0, iters=args.gemv_iters, mode=0)
        cwall = None if args.no_graph else cs.time_gemv(head=0, iters=args.gemv_iters, mode=1)[0]
        cus = cdirect if cwall is None else cwall
        cgbs = cb / cl / (cus * 1e-6) / 1e9
        log(f"gemv (code predictor, cache-resident): {cl} launches/step, {cus:.2f} "
            f"us/launch ({cgbs:.0f} GB/s), direct launches {cdirect:.2f} us")
        out["code_predictor"] = dict(launches=cl, bytes_per_launch=int(cb / cl),
                                     us_per_launch=round(cus, 3), achieved_gbs=round(cgbs, 1),
                                     direct_us_per_launch=round(cdirect, 3),
                                     graph_wall_us_per_launch=None if cwall is None
                                     else round(cwall, 3))
    return out


# algorithmic weight bytes of one frame step: talker layers + head, and 15
# code-predictor forwards each with its head (Q8_0, 34 bytes per 32 weights)
FRAME_WEIGHT_BYTES = 1759083520
# the same in f32 (4 bytes per weight; norm vectors included)
F32_FRAME_WEIGHT_BYTES = 6619626496
KV_BYTES_PER_POSITION = {"f32": 229376, "f16": 114688}  # talker, 28 layers
B32_STREAMS, B32_FRAMES = 32, 128
CONFIG2_FRAMES = 156


def batched_b32(dev, f32, tables, args):
    """Batched serving (32 streams, prompt lengths uniform in [16, 256]
    seeded, 128 frames, Q8_0 weights, activations quantized per 32-block so
    the products run on the int8 matrix cores): whole-job frames/s with the
    codes of all streams in host memory after each step, and the algorithmic
    HBM bytes of a step (the weights once, the talker K/V of every stream at
    its context length; the code predictor's K/V is under 1 % and left out)
    over the step time."""
    n, steps, warmup = B32_STREAMS, B32_FRAMES, 3
    pre = prompts(args.seed, "frame_b32", n)
    lens = np.array([p.shape[0] for p in pre])
    max_pos = int(lens.max()) + steps + warmup + 8
    kv = "f16" if args.kv16 else "f32"
    t0 = time.time()
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=q3h.Q8_0, kv_f16=int(args.kv16), act_q8=1,
                             max_positions=max_pos), f32["tl"], f32["tf"], q3h.F32)
    cs = q3h.Stack(dev, dict(synth.PREDICTOR, dtype=q3h.Q8_0, kv_f16=int(args.kv16), act_q8=1,
                             max_positions=16), f32["cl"], f32["cf"], q3h.F32)
    ts.add_head(f32["th"], q3h.F32)
    for h in f32["ch"]:
        cs.add_head(h, q3h.F32)
    frame = q3h.Frame(ts, cs, tables["codec_emb"], tables["pred_emb"], tables["tts_pad"],
                      n_streams=n, max_positions=max_pos, max_frames=steps + warmup + 8,
                      use_graph=not args.no_graph)
    log(f"batched b32: int8 stacks on the device in {time.time() - t0:.1f} s")
    total, lat, codes = run_gpu(frame, pre, steps, warmup)
    prefill_s = run_gpu.prefill_s
    seq_s = start_one_by_one(frame, pre)
    fps = n * steps / total
    # positions read per step, averaged over the steps (the row's own included)
    positions = float(np.mean([np.sum(lens + i + 1) for i in range(steps)]))
    step_bytes = FRAME_WEIGHT_BYTES + KV_BYTES_PER_POSITION[kv] * positions
    gbs = step_bytes / (total / steps) / 1e9
    out = dict(frames_per_s=round(fps, 2), streams=n, frames=steps,
               ms_per_step=round(1e3 * total / steps, 4),
               step_us_p50=round(1e6 * float(np.median(lat)), 1),
               step_us_p99=round(1e6 * float(np.percentile(lat, 99)), 1),
               prefill_ms=round(1e3 * prefill_s, 2),
               prefill="32 streams started together (q3h_frame_start_batch)",
               prefill_one_by_one_ms=round(1e3 * seq_s, 2),
               prompt_rows="U[16,256] (seeded)", activations="q8_0 (int8 MFMA)", kv=kv,
               hbm_bytes_per_step=int(step_bytes), hbm_gbs=round(gbs, 1),
               hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
    log(f"batched b32: {fps:.1f} frames/s, {1e3 * total / steps:.3f} ms per step, "
        f"{gbs:.0f} GB/s algorithmic; prefill {1e3 * prefill_s:.1f} ms ({1e3 * seq_s:.1f} ms "
        "one by one)")
    frame.destroy()
    ts.destroy()
    cs.destroy()
    if not args.no_cpu:
        cpu, nf, equal = cpu_baseline(f32, tables, pre, codes, args.cpu_seconds / 2, steps, 1)
        out["cpu_baseline"] = cpu
        out["parity"] = dict(frames=nf, codes_equal_stream0=bool(equal))
    return out


F32_B8_STREAMS, F32_B8_FRAMES = 8, 64


def f32_batch8(dev, f32, tables, args):
    """The f32-weight path at batch 8 (the reference's /f32 mode): both stacks
    and their heads in f32 on the device, 8 streams each prefilled with 512
    N(0, 1) prompt rows (causal prefill attention, products on the split-bf16
    matrix cores), then F32_B8_FRAMES frames of the 8 streams with f32
    activations and f32 K/V. Reports the timed 8 x 512-row prefill, frames/s
    over the frames with the codes of all streams in host memory after each
    step, the algorithmic HBM bytes of a step (the f32 weights once, the
    talker K/V of every stream) over the step time, stream 0's codes against
    the oracle's f32 frame step, and the oracle's rate on the host cores."""
    n, steps, warmup = F32_B8_STREAMS, F32_B8_FRAMES, 2
    pre = prompts(args.seed, "f32_b8", n)
    max_pos = F32_PROMPT_ROWS + steps + warmup + 8
    t0 = time.time()
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=q3h.F32, kv_f16=0, act_q8=0,
                             max_positions=max_pos), f32["tl"], f32["tf"], q3h.F32)
    cs = q3h.Stack(dev, dict(synth.PREDICTOR, dtype=q3h.F32, kv_f16=0, act_q8=0,
                             max_positions=16), f32["cl"], f32["cf"], q3h.F32)
    ts.add_head(f32["th"], q3h.F32)
    for h in f32["ch"]:
        cs.add_head(h, q3h.F32)
    frame = q3h.Frame(ts, cs, tables["codec_emb"], tables["pred_emb"], tables["tts_pad"],
                      n_streams=n, max_positions=max_pos, max_frames=steps + warmup + 8,
                      use_graph=not args.no_graph)
    log(f"f32 b8: f32 stacks on the device in {time.time() - t0:.1f} s "
        f"({(ts.bytes + cs.bytes) / 1e9:.2f} GB of layers)")
    total, lat, codes = run_gpu(frame, pre, steps, warmup)
    prefill_s = run_gpu.prefill_s
    seq_s = start_one_by_one(frame, pre)
    fps = n * steps / total
    positions = float(np.mean([n * (F32_PROMPT_ROWS + i + 1) for i in range(steps)]))
    step_bytes = F32_FRAME_WEIGHT_BYTES + KV_BYTES_PER_POSITION["f32"] * positions
    gbs = step_bytes / (total / steps) / 1e9
    out = dict(frames_per_s=round(fps, 2), streams=n, frames=steps,
               ms_per_step=round(1e3 * total / steps, 4),
               step_us_p50=round(1e6 * float(np.median(lat)), 1),
               step_us_p99=round(1e6 * float(np.percentile(lat, 99)), 1),
               prefill_ms=round(1e3 * prefill_s, 2),
               prefill="8 streams x 512 prompt rows started together (q3h_frame_start_batch: "
                       "the prefills overlap on the device)",
               prefill_one_by_one_ms=round(1e3 * seq_s, 2),
               prompt_rows=F32_PROMPT_ROWS, weights="f32", activations="f32", kv="f32",
               hbm_bytes_per_step=int(step_bytes), hbm_gbs=round(gbs, 1),
               hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
    log(f"f32 b8: {fps:.1f} frames/s, {1e3 * total / steps:.3f} ms per step, prefill of 8 x "
        f"512 rows {1e3 * prefill_s:.1f} ms ({1e3 * seq_s:.1f} ms one by one), {gbs:.0f} GB/s "
        "algorithmic")
    frame.destroy()
    ts.destroy()
    cs.destroy()
    if not args.no_cpu:
        cpu, nf, equal = cpu_baseline(f32, tables, pre, codes, args.cpu_seconds / 2, steps, 0,
                                      f32w=True)
        out["cpu_baseline"] = cpu
        out["parity"] = dict(frames=nf, codes_equal_stream0=bool(equal))
    return out


def talker_decode_b1(dev, ts, f32, tables, seed, args, steps=64, rows=PROMPT_ROWS):
    """Talker-only greedy decode at batch 1 (Q8_0 weights, f32 K/V): a
    48-row prefill of N(0, 1) rows, then 64 steps whose input is the codec
    embedding of the argmax of the 3072-code head (q3h_forward_embeds per
    step: host row in, logits out, so the rate includes PCIe)."""
    ctx = q3h.Context(ts, rows + steps + 8)
    codec = tables["codec_emb"]
    pre = synth.prompt(seed + 9, rows)
    codes = []
    lg, _ = ctx.forward(pre, head=0, want_normed=False)
    lat = np.empty(steps)
    t0 = time.perf_counter()
    for i in range(steps):
        a = time.perf_counter()
        c = int(np.argmax(lg))
        codes.append(c)
        lg, _ = ctx.forward(codec[c][None], head=0, want_normed=False)
        lat[i] = time.perf_counter() - a
    total = time.perf_counter() - t0
    ctx.destroy()
    out = dict(steps=steps, prompt_rows=rows, steps_per_s=round(steps / total, 1),
               step_us_p50=round(1e6 * float(np.median(lat)), 1),
               step_us_p99=round(1e6 * float(np.percentile(lat, 99)), 1),
               note="host row in and 3072 logits out per step (PCIe-inclusive)")
    log(f"talker decode b1: {steps / total:.0f} steps/s, p50 {1e6 * np.median(lat):.0f} us")
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import q3o  # the oracle, timed as the CPU baseline
        q = q3o.quantize_q8_0
        ot = q3o.Stack(synth.TALKER, [{k: (q(v) if k.startswith("w") else v)
                                       for k, v in L.items()} for L in f32["tl"]],
                       f32["tf"], q3o.Q8_0)
        th = q(f32["th"])
        sweep, equal, n_max = [], True, 0
        for threads in cpu_thread_counts():
            q3o.set_threads(threads)
            oc = q3o.Ctx(ot, rows + steps + 8)
            st = oc.forward(pre)
            n = 0
            t0 = time.perf_counter()
            while n < steps and (n < 2 or time.perf_counter() - t0 < args.cpu_seconds / 4):
                c = int(np.argmax(ot.head(th, st)))
                equal = equal and c == codes[n]
                st = oc.forward(codec[c][None])
                n += 1
            dt = time.perf_counter() - t0
            oc.destroy()
            n_max = max(n_max, n)
            sweep.append(dict(threads=threads, steps_per_s=round(n / dt, 3), steps=n))
            log(f"talker decode on the CPU: {n / dt:.2f} steps/s on {threads} threads")
        ot.destroy()
        best = max(sweep, key=lambda r: r["steps_per_s"])
        out["cpu_baseline"] = dict(value=best["steps_per_s"], unit="steps/s",
                                   cores=best["threads"], kind="port",
                                   sample=f"the first steps of the same decode (oracle, C + "
                                          f"OpenMP), about {args.cpu_seconds / 4:.0f} s per "
                                          "thread count", threads_sweep=sweep, **cpu_info())
        out["parity"] = dict(steps=n_max, codes_equal=bool(equal))
    return out


LONG_LENGTHS = (2048, 4096, 8192)


def long_context_attention(dev, f32, tables, seed, steps=32, iters=10):
    """Talker Q8_0 at batch 1 with an f16 K/V cache prefilled to 2048, 4096 and
    8192 positions (N(0,1) values from a seed): 32 greedy decode steps at each
    length (q3h_forward_embeds, host row in and logits out, so PCIe-inclusive),
    then the decode attention kernels alone (launched directly over the 28
    layers, iters passes between two events on their stream, so the gaps
    between the split kernel, the merge and the next layer count too):
    algorithmic bytes = the f16 K/V of every position read once (8 kv heads x
    128 dims x 2 x 2 B = 4 KB per position and layer)."""
    t0 = time.time()
    cap = max(LONG_LENGTHS) + steps + 8
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=q3h.Q8_0, kv_f16=1, act_q8=0,
                             max_positions=cap), f32["tl"], f32["tf"], q3h.F32)
    ts.add_head(f32["th"], q3h.F32)
    codec = tables["codec_emb"]
    rng = np.random.Generator(np.random.PCG64(seed + 77))
    shape = (synth.TALKER["layers"], synth.TALKER["kv_heads"])
    out = []
    for L in LONG_LENGTHS:
        k = rng.standard_normal(shape + (L, 128), dtype=np.float32)
        v = rng.standard_normal(shape + (L, 128), dtype=np.float32)
        ctx = q3h.Context(ts, cap)
        ctx.fill_kv(k, v)
        del k, v
        x = synth.prompt(seed + L, 1)
        lat = np.empty(steps)
        for i in range(steps):
            a = time.perf_counter()
            lg, _ = ctx.forward(x, head=0, want_normed=False)
            lat[i] = time.perf_counter() - a
            x = codec[int(np.argmax(lg[:2048]))][None]
        us, nbytes = ctx.time_attention(iters=iters)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append(dict(positions=ctx.length, attention_us_per_layer=round(us, 3),
                        attention_bytes_per_layer=int(nbytes), attention_gbs=round(gbs, 1),
                        frac=round(gbs / HBM_PEAK_GBS, 4),
                        decode_step_us_p50=round(1e6 * float(np.median(lat)), 1)))
        log(f"long context {L}: attention {us:.2f} us/layer ({gbs:.0f} GB/s), "
            f"decode step p50 {1e6 * np.median(lat):.0f} us")
        ctx.destroy()
    ts.destroy()
    log(f"long-context attention in {time.time() - t0:.1f} s")
    return dict(kernel="k_attn_split + k_attn_merge (f16 K/V, talker decode, per layer)",
                kv="f16", steps_per_length=steps, results=out)


SHORT_LENGTHS = (64, 126, 192, 256)


def short_context_attention(dev, f32, seed, iters=20):
    """The frame's talker decode attention at batch 1 (Q8_0 talker, f32 K/V,
    the frame's cache type) with the cache filled to 63, 125, 191 and 255
    positions (N(0,1) values from a seed), so that the new row is position 64,
    126 (the 156-frame pass's average context), 192 and 256: the attention
    kernel of the 28 layers launched directly iters times between two events
    on its stream (gaps included); algorithmic bytes = the f32 K/V of every
    cached position read once (8 kv heads x 128 dims x 2 x 4 B = 8 KB per
    position and layer) + the new key and value, the q / k / v row and the
    output."""
    cap = max(SHORT_LENGTHS) + 8
    ts = q3h.Stack(dev, dict(synth.TALKER, dtype=q3h.Q8_0, kv_f16=0, act_q8=0,
                             max_positions=cap), f32["tl"], f32["tf"], q3h.F32)
    rng = np.random.Generator(np.random.PCG64(seed + 78))
    shape = (synth.TALKER["layers"], synth.TALKER["kv_heads"])
    out = []
    for L in SHORT_LENGTHS:
        k = rng.standard_normal(shape + (L - 1, 128), dtype=np.float32)
        v = rng.standard_normal(shape + (L - 1, 128), dtype=np.float32)
        ctx = q3h.Context(ts, cap)
        ctx.fill_kv(k, v)
        us, nbytes = ctx.time_attention(iters=iters)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append(dict(positions=L, attention_us_per_layer=round(us, 3),
                        attention_bytes_per_layer=int(nbytes), attention_gbs=round(gbs, 1),
                        frac=round(gbs / HBM_PEAK_GBS, 4)))
        log(f"short context {L}: attention {us:.2f} us/layer ({gbs:.0f} GB/s)")
        ctx.destroy()
    ts.destroy()
    return dict(kernel="k_attn_short (f32 K/V, talker decode at batch 1, per layer)", kv="f32",
                results=out)


def codec_macs_per_frame():
    """Multiply-adds of the decoder's back part per frame (every convolution:
    rows per frame x taps x in x out; transposed convolutions as the causal
    convolutions the library runs)."""
    L, D = synth.CODEC_LATENT, synth.CODEC_DIM
    m = 1 * L * 2 * L + 2 * L * 2 * L  # two transposed convolutions 2 / 2
    m += (2 + 4) * (2 * L * 4 * L + 7 * L)  # ConvNeXt pointwise pair + depthwise
    m += 4 * 7 * L * D  # input convolution
    rows = 4
    for i, rate in enumerate(synth.CODEC_RATES):
        cin, cout = D >> i, D >> (i + 1)
        m += rows * 2 * cin * rate * cout  # transposed convolution, 2 taps
        rows *= rate
        m += 3 * rows * (7 * cout * cout + cout * cout)  # residual units
    return m + rows * 7 * (D >> 4)


def codec_back(dev, seed, frames=156, cpu=True):
    """The 12 Hz decoder's back part (TQwenCodecVulkan.Back): `frames` frames of
    N(0,1) transformer rows decoded in passes of 16 frames (the reference's
    CHUNK_FRAMES) and one frame per call (streaming), host rows in and PCM out;
    frames/s, real-time factor at 12.5 frames per second, and the matrix-core
    rate (2 x multiply-adds / time against the f32 peak)."""
    w = synth.codec_weights(seed)
    c = q3h.Codec(dev, w, max_frames=16)
    x = synth.prompt(seed + 90, frames)
    macs = codec_macs_per_frame()
    out = dict(frames=frames, macs_per_frame=int(macs))
    for name, step in (("passes_of_16", 16), ("one_frame_per_call", 1)):
        c.reset()
        c.back(x[:step])  # warm-up
        c.reset()
        t0 = time.perf_counter()
        for f in range(0, frames, step):
            c.back(x[f:f + step])
        dt = time.perf_counter() - t0
        fps = frames / dt
        tf = 2 * macs * fps / 1e12
        out[name] = dict(frames_per_s=round(fps, 1), ms_per_frame=round(1e3 / fps, 3),
                         real_time_factor=round(fps / 12.5, 1), tflops=round(tf, 2),
                         mfma_frac=round(tf / F32_MFMA_PEAK_TFLOPS, 4))
        log(f"codec back ({name}): {fps:.1f} frames/s, {1e3 / fps:.3f} ms per frame, "
            f"{tf:.1f} TFLOP/s")
    c.destroy()
    if cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import q3o  # the oracle, timed as the CPU baseline
        threads = min(16, len(os.sched_getaffinity(0)))
        q3o.set_threads(threads)
        oc = q3o.Codec(w)
        n = 2
        t0 = time.perf_counter()
        oc.back(x[:n])
        dt = time.perf_counter() - t0
        oc.destroy()
        out["cpu_baseline"] = dict(value=round(n / dt, 3), unit="frames/s", cores=threads,
                                   kind="port", sample=f"{n} frames, oracle back part "
                                   "(C + OpenMP, double sums)")
        log(f"codec back on the CPU (oracle): {n / dt:.2f} frames/s")
    return out


TEXT_VOCAB_BENCH = 16384  # rows of the synthetic text table (one row gathered per token)
TEXT_TOKENS = 40


def start_ids(seed, n_text):
    """PromptIds (talker.pas:430-452) of a sentence of n_text tokens: im_start,
    assistant, \\n, the text, im_end, \\n, im_start, assistant, \\n; the codec
    ids of the Auto language with no speaker (nothink, think_bos, think_eos,
    codec_pad, codec_bos, talker.pas:512-521) and the special ids."""
    rng = np.random.Generator(np.random.PCG64(seed + 55))
    text = rng.integers(0, TEXT_VOCAB_BENCH - 16, n_text).tolist()
    im_start, im_end, assistant, nl = TEXT_VOCAB_BENCH - 1, TEXT_VOCAB_BENCH - 2, 77, 198
    ids = [im_start, assistant, nl] + text + [im_end, nl, im_start, assistant, nl]
    special = dict(tts_bos=TEXT_VOCAB_BENCH - 5, tts_eos=TEXT_VOCAB_BENCH - 4,
                   tts_pad=TEXT_VOCAB_BENCH - 3, codec_pad=2148, codec_bos=2149)
    return ids, [2155, 2156, 2157, 2148, 2149], special


def start_from_text(dev, ts, cs, tables, seed, max_pos, iters=10, use_graph=True):
    """Time to the first frame from token ids (TQwenTalker.Start then the first
    NextFrame): q3h_frame_start_text projects the prompt's 48 text rows
    (TextProject, fc1 2048 x 2048 + SiLU + fc2 2048 -> 1024 in f32 on the matrix
    cores), assembles the prefill and trailing rows on the device and prefills
    the talker; then one frame step. Wall clock, host ids in and codes out;
    median of iters after 2 warm-ups, non-streaming (49 prefill rows) and
    streaming (8 prefill rows + 40 trailing). Also the projection alone
    (q3h_text_project of the 48 ids, host ids in, host rows out)."""
    emb, w1, b1, w2, b2 = synth.text_projection(seed, TEXT_VOCAB_BENCH)
    proj = q3h.TextProj(dev, emb, w1, b1, w2, b2)
    fr = q3h.Frame(ts, cs, tables["codec_emb"], tables["pred_emb"], tables["tts_pad"],
                   n_streams=1, max_positions=max_pos, max_frames=64, use_graph=use_graph)
    ids, codec, sp = start_ids(seed, TEXT_TOKENS)
    out = dict(text_tokens=TEXT_TOKENS, prompt_ids=len(ids), text_vocab=TEXT_VOCAB_BENCH)
    for ns in (True, False):
        st, ff = [], []
        for i in range(iters + 2):
            a = time.perf_counter()
            fr.start_text(0, proj, ids, codec, non_streaming=ns, **sp)
            b = time.perf_counter()
            fr.step()
            c = time.perf_counter()
            if i >= 2:
                st.append(b - a)
                ff.append(c - a)
        key = "non_streaming" if ns else "streaming"
        out[key] = dict(start_ms_p50=round(1e3 * float(np.median(st)), 3),
                        first_frame_ms_p50=round(1e3 * float(np.median(ff)), 3))
        log(f"start from text ({key}): start {1e3 * np.median(st):.2f} ms, "
            f"first frame {1e3 * np.median(ff):.2f} ms")
    pid = np.array(ids, np.int32)
    lat = []
    for i in range(iters + 2):
        a = time.perf_counter()
        proj.project(pid)
        if i >= 2:
            lat.append(time.perf_counter() - a)
    out["project_48_rows_us_p50"] = round(1e6 * float(np.median(lat)), 1)
    log(f"text projection of {len(ids)} rows: {1e6 * np.median(lat):.0f} us")
    fr.destroy()
    proj.destroy()
    start_from_text.tables = (emb, w1, b1, w2, b2)
    start_from_text.ids = pid
    return out


def cpu_text_projection(tables, ids, budget_s=2.0):
    """The oracle's TextProject of the same ids on the host cores (the
    reference's CPU text projection), timed until budget_s is spent."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import q3o  # the oracle, timed as the CPU baseline

    threads = min(16, len(os.sched_getaffinity(0)))
    q3o.set_threads(threads)
    n = 0
    t0 = time.perf_counter()
    while n < 2 or time.perf_counter() - t0 < budget_s:
        q3o.text_project(*tables, ids)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return dict(value=round(1e6 * dt, 1), unit="us per projection", cores=threads, kind="port",
                sample=f"TextProject of {len(ids)} ids (oracle, C + OpenMP), {n} runs")


COPY_BYTES = 256 << 20


def copy_calibration(iters=5):
    """A plain copy of COPY_BYTES (read once, written once) by an elementwise
    kernel, iters times: the bytes the FETCH_SIZE / WRITE_SIZE counters report
    per dispatch of it scale the counters of the kernels under study."""
    import torch
    x = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(iters):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": COPY_BYTES, "copy_bytes_written": COPY_BYTES,
                      "dispatches": iters}), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["frame_b1", "frame_b32", "f32_b8"], default="frame_b1")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--gemv-iters", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="seconds of oracle frames per thread count (CPU baseline)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the kernels directly instead of replaying hipGraphs "
                         "(for tracers that do not follow graph capture)")
    ap.add_argument("--no-long-attn", action="store_true",
                    help="skip the long-context attention measurement (frame_b1)")
    ap.add_argument("--no-text", action="store_true",
                    help="skip the time-to-first-frame measurement from token ids (frame_b1)")
    ap.add_argument("--kv16", action="store_true",
                    help="K/V caches in half floats (the reference's KvF16 option, lm.pas:353); "
                         "the default is its f32 cache")
    ap.add_argument("--no-b32", action="store_true",
                    help="skip the 32-stream int8 sub-record of the default run")
    ap.add_argument("--no-f32", action="store_true",
                    help="skip the f32-weight batch-8 sub-record of the default run")
    ap.add_argument("--no-talker", action="store_true",
                    help="skip the talker-only decode sub-record of the default run")
    ap.add_argument("--no-codec", action="store_true",
                    help="skip the decoder back-part measurement (frame_b1)")
    ap.add_argument("--codec-only", action="store_true",
                    help="only the decoder back-part measurement (profiling runs)")
    ap.add_argument("--no-roofline", action="store_true",
                    help="skip the matrix-vector roofline measurement (its kernel-attached "
                         "events are not for runs under a kernel tracer)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the matrix-vector roofline measurement (profiling runs)")
    ap.add_argument("--gemv-stack", choices=["talker", "code", "both"], default="talker",
                    help="with --gemv-only: the stack whose products are timed (code: the "
                         "code predictor)")
    ap.add_argument("--gemv-mode", type=int, choices=[0, 1, 2], default=2,
                    help="with --gemv-only: 0 direct launches (tracers, counters), 1 graph "
                         "replay, 2 events attached to each launch")
    ap.add_argument("--long-attn-only", action="store_true",
                    help="only the long-context attention measurement (profiling runs)")
    ap.add_argument("--short-attn-only", action="store_true",
                    help="only the batch-1 talker decode attention at 64-256 positions "
                         "(profiling runs)")
    ap.add_argument("--prompt-rows", type=int, default=PROMPT_ROWS,
                    help="frame_b1: prompt rows of the prefill (profiling the prefill products "
                         "at other sizes; the measured workload is 48)")
    ap.add_argument("--copy-only", action="store_true",
                    help="only a plain copy kernel of known size (calibrates the FETCH_SIZE "
                         "and WRITE_SIZE counters of profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this library runs on one GPU; --gpus {args.gpus} is not supported "
              "(independent streams would shard across GPUs with no exchange)", file=sys.stderr)
        return 2
    if args.copy_only:
        return copy_calibration()
    if args.codec_only:
        if not q3h.available():
            raise RuntimeError("no gfx950 device")
        dev = q3h.Device(0)
        print(json.dumps({"codec_back": codec_back(dev, args.seed, cpu=False)}), flush=True)
        dev.close()
        return 0
    if args.short_attn_only:
        if not q3h.available():
            raise RuntimeError("no gfx950 device")
        dev = q3h.Device(0)
        tl, tf = synth.stack_weights(args.seed, "talker.model.", synth.TALKER)
        print(json.dumps({"decode_attention_b1":
                          short_context_attention(dev, dict(tl=tl, tf=tf), args.seed)}),
              flush=True)
        dev.close()
        return 0
    if args.long_attn_only:
        if not q3h.available():
            raise RuntimeError("no gfx950 device")
        dev = q3h.Device(0)
        tl, tf = synth.stack_weights(args.seed, "talker.model.", synth.TALKER)
        f32 = dict(tl=tl, tf=tf, th=synth.talker_head(args.seed))
        tables = dict(codec_emb=synth.codec_embedding(args.seed))
        print(json.dumps({"long_context_attention":
                          long_context_attention(dev, f32, tables, args.seed)}), flush=True)
        dev.close()
        return 0
    b1 = args.workload == "frame_b1"
    f32w = args.workload == "f32_b8"
    n = 1 if b1 else (8 if f32w else 32)
    steps = args.steps if args.steps is not None else (156 if b1 else (256 if f32w else 128))
    warmup = args.warmup
    if not q3h.available():
        raise RuntimeError("no gfx950 device")
    pre = prompts(args.seed, args.workload, n, args.prompt_rows)
    maxlen = max(p.shape[0] for p in pre)
    max_pos = maxlen + max(steps, warmup, CONFIG2_FRAMES if b1 else 0) + 8
    dev = q3h.Device(0)
    act_q8 = 0 if (b1 or f32w) else 1
    ts, cs, tables, f32 = build_model(dev, args.seed, max_pos, act_q8,
                                      q3h.F32 if f32w else q3h.Q8_0, int(args.kv16))
    if args.gemv_only:
        # the products of one decode step of the chosen stack(s), iters times
        # (mode 0 direct launches for kernel tracers and counters, 1 graph
        # replay, 2 events attached to each launch)
        out = {}
        for name, st in (("talker", ts), ("code_predictor", cs)):
            if args.gemv_stack not in (name.split("_")[0], "both"):
                continue
            us, n_l, nb = st.time_gemv(head=0, iters=args.gemv_iters, mode=args.gemv_mode)
            out[name] = dict(launches=n_l, bytes_per_launch=int(nb / n_l),
                             us_per_launch=round(us, 3), mode=args.gemv_mode)
            log(f"gemv {name}: {n_l} launches, {us:.2f} us per launch (mode {args.gemv_mode})")
        print(json.dumps({"gemv": out}), flush=True)
        ts.destroy()
        cs.destroy()
        dev.close()
        return 0
    frame = q3h.Frame(ts, cs, tables["codec_emb"], tables["pred_emb"], tables["tts_pad"],
                      n_streams=n, max_positions=max_pos,
                      max_frames=max(steps, warmup, CONFIG2_FRAMES) + 8,
                      use_graph=not args.no_graph)
    log(f"{args.workload}: {n} stream(s), warm-up {warmup}, timing {steps} steps")
    total, lat, codes = run_gpu(frame, pre, steps, warmup)
    prefill_s = run_gpu.prefill_s
    fps = n * steps / total
    log(f"{fps:.1f} frames/s, {1e3 * total / steps:.3f} ms per step "
        f"(p50 {1e6 * np.median(lat):.0f} us, p99 {1e6 * np.percentile(lat, 99):.0f} us); "
        f"prefill of {n} stream(s) {1e3 * prefill_s:.1f} ms")

    full = None
    if b1 and steps != CONFIG2_FRAMES:
        # the whole sentence of the configuration (context 48 -> 204)
        f_total, f_lat, _ = run_gpu(frame, pre, CONFIG2_FRAMES, 0)
        full = dict(frames=CONFIG2_FRAMES, frames_per_s=round(CONFIG2_FRAMES / f_total, 2),
                    ms_per_step=round(1e3 * f_total / CONFIG2_FRAMES, 4),
                    step_us_p50=round(1e6 * float(np.median(f_lat)), 1))
        log(f"{CONFIG2_FRAMES} frames: {full['frames_per_s']:.1f} frames/s")

    roofline = gemv_roofline(ts, args, cs if b1 else None) \
        if not (f32w or args.no_roofline) else None

    # the same frames drawn with the qwen_tts default sampling (temperature 0.9,
    # top-k 50 on both choosers, talker.pas:208-216): the sampler's cost
    frame.set_sampling(True, 0.9, 50, 1.0, True, 0.9, 50, 1.0, seed=args.seed + 1)
    s_total, s_lat, _ = run_gpu(frame, pre, steps, warmup)
    frame.set_sampling()
    sampled = dict(frames_per_s=round(n * steps / s_total, 2),
                   ms_per_step=round(1e3 * s_total / steps, 4),
                   step_us_p50=round(1e6 * float(np.median(s_lat)), 1),
                   sampling="temperature 0.9, top-k 50, top-p 1 (talker and code predictor)")
    log(f"sampled: {sampled['frames_per_s']:.1f} frames/s, {sampled['ms_per_step']:.3f} ms per step")

    frame.destroy()
    talker_b1 = talker_decode_b1(dev, ts, f32, tables, args.seed, args) \
        if (b1 and not args.no_talker) else None
    b32 = batched_b32(dev, f32, tables, args) if (b1 and not args.no_b32) else None
    f32b8 = f32_batch8(dev, f32, tables, args) if (b1 and not args.no_f32) else None
    load = load_from_bf16(dev, f32, act_q8) if b1 else None
    text_start = None
    if b1 and not args.no_text:
        text_start = start_from_text(dev, ts, cs, tables, args.seed, max_pos,
                                     use_graph=not args.no_graph)
    codec = None
    if b1 and not args.no_codec:
        codec = codec_back(dev, args.seed, cpu=not args.no_cpu)
    long_attn = None
    short_attn = None
    if b1 and not args.no_long_attn:
        short_attn = short_context_attention(dev, f32, args.seed)
        long_attn = long_context_attention(dev, f32, tables, args.seed)

    cpu = None
    parity = None
    if not args.no_cpu:
        cpu, nf, equal = cpu_baseline(f32, tables, pre, codes, args.cpu_seconds, steps, act_q8,
                                      f32w)
        parity = dict(frames=nf, codes_equal_stream0=bool(equal))
        log(f"cpu baseline: {cpu['value']:.2f} frames/s on {cpu['cores']} threads; "
            f"codes equal over {nf} frames: {equal}")
        if text_start is not None:
            text_start["cpu_baseline"] = cpu_text_projection(start_from_text.tables,
                                                             start_from_text.ids)
            log(f"cpu text projection: {text_start['cpu_baseline']['value']:.0f} us")
    ts.destroy()
    cs.destroy()
    dev.close()

    out = {
        "metric": "talker+CP frames/s @B=1 & B=32 (Q8_0); frame-step µs; "
                  "% HBM/MFMA roofline",
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(1e3 * total / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) prompt embeddings)",
        "config": {"workload": args.workload, "graph": not args.no_graph, "streams": n, "prompt_rows":
                   args.prompt_rows if b1 else (F32_PROMPT_ROWS if f32w else "U[16,256]"),
                   "frames": steps, "talker_layers": 28, "cp_layers": 5, "hidden": 1024,
                   "heads": "16q/8kv x 128", "ffn": 3072, "weights": "f32" if f32w else "Q8_0",
                   "kv": "f16" if args.kv16 else "f32", "activations": "q8_0 (int8 MFMA)" if act_q8 else "f32"},
        "prefill_ms": round(1e3 * prefill_s, 2),
        "step_us_p50": round(1e6 * float(np.median(lat)), 1),
        "step_us_p99": round(1e6 * float(np.percentile(lat, 99)), 1),
        "frame_b1_156_frames": full,
        "batched_b32": b32,
        "f32_b8": f32b8,
        "talker_decode_b1": talker_b1,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
        "decode_attention_b1": short_attn,
        "long_context_attention": long_attn,
        "start_from_text": text_start,
        "sampled": sampled,
        "load_from_bf16": load,
        "codec_back": codec,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
