"""Benchmark: stories110M-shaped fp32 greedy decode on one MI355X.

One step = one full greedy decode of the 1024-position context (BASELINE
config 4): pt_generate over token ids (prompt forcing, then argmax), each
position one launch of the device-resident pt_forward_step (85 projections +
attention + argmax as one kernel, the library's default decode path; graphs
of 8 positions), positions 0..1023 of the KV cache, synthetic random-init
weights ~N(0, 0.02).  `value` = decoded tokens per second over the K timed
decodes.

Prints ONE JSON line: decode tok/s as `value`, the dominant kernel's HBM
roofline (per-launch HIP-event timing of eager steps over all 1024
positions, algorithmic bytes per launch, counter-measured HBM traffic), the
same decode on the captured multi-kernel path for comparison, and the
reference's own CPU decode timed on a bounded sample, pinned to one core.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_stories110M_hbm_traffic.md")
TRAIN_PROFILE = os.path.join(ROOT, "profiles", "train_stories15M_T256_kernel_stats.md")


# The sources of the decode kernels: a traffic figure measured on other
# sources says nothing about this build.
DECODE_SOURCES = ["pitorch_amd/csrc/ptmi_decode_step.hip", "pitorch_amd/csrc/ptmi_decode.hip",
                  "pitorch_amd/csrc/ptmi_matvec.hip", "pitorch_amd/csrc/ptmi_core.hip",
                  "pitorch_amd/csrc/ptmi_internal.h", "pitorch_amd/csrc/ptmi_model.h"]


def sources_hash(files, root=ROOT):
    """First 16 hex digits of the SHA-256 over the given sources, in order."""
    import hashlib
    h = hashlib.sha256()
    for rel in files:
        with open(os.path.join(root, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def decode_sources_hash(root=ROOT):
    """sources_hash of the decode kernels' sources (DECODE_SOURCES)."""
    return sources_hash(DECODE_SOURCES, root)


# The sources of the training step's kernels (for the in-step kernel times
# a committed kernel trace measured).
TRAIN_SOURCES = ["pitorch_amd/csrc/ptmi_train.hip", "pitorch_amd/csrc/ptmi_gemm.hip",
                 "pitorch_amd/csrc/ptmi_internal.h", "pitorch_amd/csrc/ptmi_model.h"]


def train_sources_hash(root=ROOT):
    """sources_hash of the training kernels' sources (TRAIN_SOURCES)."""
    return sources_hash(TRAIN_SOURCES, root)


def _profile_row(kind, tag, role, path, sources):
    """(cells, note) of the committed profile row `| kind | tag | role |
    <sources hash> | ... |` in `path`: the row's cells when it was measured
    on the sources with hash `sources`; otherwise None and why."""
    try:
        lines = open(path).read().splitlines()
    except OSError:
        return None, f"no profile at {os.path.relpath(path, ROOT)}"
    for ln in lines:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == kind and cells[1] == tag and cells[2] == role:
            if cells[3].strip("`") != sources:
                return None, (f"the committed {kind} row was measured on sources {cells[3].strip('`')}, "
                              f"this build's are {sources}")
            return cells, None
    return None, f"no {kind} row for {tag} {role}"


def committed_traffic(role, workload_tag, path=TRAFFIC_PROFILE, sources=None):
    """(HBM bytes per launch of decode kernel `role`, note): the figure the
    two rocprofv3 FETCH_SIZE / WRITE_SIZE passes committed in `path` measured
    (rows `| traffic | <tag> | <role> | <sources hash> | ... | <bytes> |`),
    when the row was measured on the decode sources of this build (hash
    `sources`, default: this tree's); otherwise None and why."""
    cells, note = _profile_row("traffic", workload_tag, role, path, sources or decode_sources_hash())
    if cells is None:
        return None, note
    try:
        return int(cells[-1]), None
    except ValueError:
        return None, "unreadable traffic row"


def committed_in_step(path=TRAIN_PROFILE, sources=None):
    """({"steps", "gemm_ms", "kernels_ms"}, note): the training step's summed
    kernel durations per step, of its GEMM kernels and of all its kernels,
    from the eager kernel trace committed in `path` (row `| in-step |
    stories15M T256 | step | <sources hash> | <steps> | <GEMM µs> | <all µs>
    |`), when it was measured on this build's training sources; otherwise
    None and why."""
    cells, note = _profile_row("in-step", "stories15M T256", "step", path, sources or train_sources_hash())
    if cells is None:
        return None, note
    try:
        return {"steps": int(cells[4]), "gemm_ms": float(cells[5]) / 1e3, "kernels_ms": float(cells[6]) / 1e3}, None
    except (ValueError, IndexError):
        return None, "unreadable in-step row"


def matvec_bytes(d, n):
    """Algorithmic bytes of y[d] = W[d,n] x[n]: 4*(d*n + n + d)."""
    return 4 * (d * n + n + d)


def role_bytes(cfg, positions):
    """Algorithmic bytes per launch of each decode kernel, averaged over the
    given positions (attention reads K and V rows 0..pos of every head)."""
    D, H, _, NH, _, V, _ = cfg
    KV = D
    mean_ctx = sum(p + 1 for p in positions) / len(positions)
    return {
        "qkv": matvec_bytes(D + 2 * KV, D),
        "attention": int(4 * (2 * KV * mean_ctx + D)),
        "wo": matvec_bytes(D, D),
        "w13": matvec_bytes(2 * H, D),
        "w2": matvec_bytes(D, H),
        "classifier": matvec_bytes(V, D),
        "argmax": 4 * V,
        "step": int(decode_bytes_per_token(cfg, positions)),
    }


def decode_bytes_per_token(cfg, positions):
    """Weights + average KV traffic per token (4*P_proj + 8*L*D*(p+1) + 8*L*D)."""
    D, H, L, _, _, V, _ = cfg
    proj = L * (4 * D * D + 3 * H * D) + V * D
    kv = sum(8 * L * D * (p + 1) + 8 * L * D for p in positions) / len(positions)
    return 4 * proj + kv


SWEEP = [(288, 288), (768, 288), (288, 768), (32000, 288), (2048, 768), (768, 2048), (32000, 768),
         (2304, 768), (4096, 768)]


def matvec_sweep(pa, footprint_mb=1536, reps_max=2048):
    """Config 2: standalone y = W x at each shape, W rotated through a
    footprint well above the 256 MB MALL so every launch reads HBM.  The
    launches are captured back to back in a hipGraph on the library stream
    and timed with HIP events around its replay, so host launch cost is not
    in the figure.  Each shape is timed with the default kernel (x held in
    registers per wave) and with the ablation kernel that re-reads x for
    every row pass (ptmi_matvec_dev_xreread, the counterpart of the
    reference's smatvec_tmu_no_packing baseline)."""
    from pitorch_amd._hip import DeviceArray, Event, Graph
    L = pa.load_ptmi()
    stream = L.ptmi_stream()
    big = DeviceArray(footprint_mb * (1 << 20) // 4)
    x = DeviceArray.from_host(pa.seed_uniform(3, 2048))
    y = DeviceArray(32000)
    out = []
    for d, n in SWEEP:
        stride = (d * n + 63) // 64 * 64
        copies = max(1, min(big.n // stride, reps_max))
        row = {"d": d, "n": n}
        for tag, entry in (("", L.ptmi_matvec_dev), ("x_reread_", L.ptmi_matvec_dev_xreread)):
            pa._ffi.check(entry(big.ptr, n, x.ptr, y.ptr, d, n, None))
            pa._ffi.check(L.ptmi_sync())

            def enqueue():
                for i in range(copies):
                    pa._ffi.check(entry(big.ptr + 4 * i * stride, n, x.ptr, y.ptr, d, n, stream))

            g = Graph(stream, enqueue)
            g.launch()
            e0, e1 = Event(), Event()
            e0.record(stream)
            g.launch()
            e1.record(stream)
            us = e0.elapsed_ms(e1) * 1e3 / copies
            g.free()
            gbs = matvec_bytes(d, n) / (us * 1e-6) / 1e9
            row.update({tag + "us": round(us, 2), tag + "GBps": round(gbs, 1)})
            if not tag:
                row["frac"] = round(gbs / HBM_PEAK_GBS, 4)
        out.append(row)
    for a in (big, x, y):
        a.free()
    return out


class pinned_to_one_core:
    """Run the block on one host core only (the reference path is
    single-threaded; the survey's CPU baseline is `taskset -c 0`): the
    lowest-numbered core this process may use (core 0 where it is allowed)."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        self.core = min(self.saved)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)


def cpu_extra():
    """The reference's own host code (oracle/_ref, -O2 -ffp-contract=off,
    1 thread pinned to one core) on the other measured paths: its
    smatvec_cpu at every sweep shape (~0.2 s each) and one pt_train_step
    of the 15M training configuration (T=256, same blob and ids; ~10 s)."""
    import ctypes

    import numpy as np

    import pitorch_amd as pa
    from tests._oracle import P, ref
    R = ref()
    if R is None:
        return None
    sweep = []
    with pinned_to_one_core() as pin:
        for d, n in SWEEP:
            W = pa.seed_uniform(4, d * n)
            xx = pa.seed_uniform(5, n)
            yy = np.zeros(d, np.float32)
            k, t0 = 0, time.perf_counter()
            while k < 2 or time.perf_counter() - t0 < 0.2:
                R.smatvec_cpu(P(W), P(xx), P(yy), d, n)
                k += 1
            us = (time.perf_counter() - t0) * 1e6 / k
            sweep.append({"d": d, "n": n, "us": round(us, 1),
                          "GBps": round(matvec_bytes(d, n) / (us * 1e-6) / 1e9, 2)})
        cfg = pa.STORIES["stories15M"]
        blob = pa.synth_model(cfg, pa.SEED_MODEL["stories15M"])
        tok = pa.seed_tokens(pa.SEED_TRAIN, 256, cfg[5]).astype(np.int32)
        ctx = R.ref_ctx_new(P(blob), 256)
        t0 = time.perf_counter()
        R.ref_train_step(ctx, tok.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), 256, 1e-3)
        train_s = time.perf_counter() - t0
        R.ref_ctx_free(ctx)
    return {"cores": 1, "kind": "reference", "pinned": f"core {pin.core}", "matvec_sweep": sweep,
            "train_step": {"workload": "stories15M, T=256, lr=1e-3, 1 step", "s_per_step": round(train_s, 2)}}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(blob, prompt, positions):
    """The reference's own host decode (oracle/_ref: pitorch/pt.c
    pt_forward_step with smatvec_cpu, built -O2 -ffp-contract=off), one
    thread pinned to one core, on the same 110M blob and prompt: the same
    greedy decode of positions 0..positions-1 as the GPU figure (~1 minute
    on one core; the cost of a token grows with its position, so a shorter
    sample would overstate the CPU)."""
    from tests._oracle import P, ref
    R = ref()
    if R is None:
        return None
    ctx = R.ref_ctx_new(P(blob), 0)
    tok = int(prompt[0])
    n = 0
    with pinned_to_one_core() as pin:
        t0 = time.perf_counter()
        while n < positions:
            nxt = R.ref_forward_step(ctx, tok)
            tok = int(prompt[n + 1]) if n + 1 < len(prompt) else nxt
            n += 1
        dt = time.perf_counter() - t0
    R.ref_ctx_free(ctx)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": 1, "kind": "reference",
            "sample": f"positions 0..{n - 1} of the stories110M greedy decode, the GPU figure's workload (same "
                      f"blob and prompt), {dt:.1f} s, 1 thread pinned to core {pin.core} of {cpu_model()}, "
                      f"host nproc={os.cpu_count()}"}


MFMA_FP32_PEAK_TFLOPS = 157.3


def train_gemm_shapes(cfg, T):
    """Every GEMM of one pt_train_step at this config (op, M, N, K, count,
    accumulate): forward Y = X W^T (NT), backward dX = dY W (NN) and
    dW = dY^T X (TN), R = T-1 backward rows; QKV and w1|w3 are fused as in
    the device layout.  `accumulate` is what the device step does: the Wo
    and w2 forward GEMMs add the residual stream; every other GEMM writes
    (gradients are written, not accumulated into zeroed buffers)."""
    D, H, L, _, _, V, _ = cfg
    R = T - 1
    QS = 3 * D
    fwd = [(2, T, QS, D, L, 0), (2, T, D, D, L, 1), (2, T, 2 * H, D, L, 0), (2, T, D, H, L, 1), (2, T, V, D, 1, 0)]
    dx = [(0, R, D, V, 1, 0), (0, R, H, D, L, 0), (0, R, D, 2 * H, L, 0), (0, R, D, D, L, 0), (0, R, D, QS, L, 0)]
    dw = [(1, V, D, R, 1, 0), (1, D, H, R, L, 0), (1, 2 * H, D, R, L, 0), (1, D, D, R, L, 0), (1, QS, D, R, L, 0)]
    return fwd + dx + dw


def bench_train(pa, reps=20):
    """stories15M training step (config 5): ms/step of the device pt_train_step
    (hipGraph per step) and fp32-MFMA utilisation of its GEMMs; each GEMM
    shape (with the step's accumulate flag) is captured `reps` times back to
    back in a hipGraph on the library stream and timed with HIP events
    around graph replays, so host launch cost is not in the figure."""
    import numpy as np
    from pitorch_amd._hip import DeviceArray, Event, Graph

    L = pa.load_ptmi()
    name, T, lr = "stories15M", 256, 1e-3
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    tokens = pa.seed_tokens(pa.SEED_TRAIN, T, cfg[5])
    m = pa.Model(blob, max_T=T)
    for _ in range(3):                       # capture the step's graph, reach steady clocks
        m.train_step(tokens, lr)
    t0 = time.perf_counter()
    losses = [m.train_step(tokens, lr) for _ in range(18)]
    step_ms = (time.perf_counter() - t0) * 1e3 / 18
    m.close()
    stream = L.ptmi_stream()
    shapes = train_gemm_shapes(cfg, T)
    maxA = max(M * K for _, M, N, K, _, _ in shapes)
    maxB = max(K * N for _, M, N, K, _, _ in shapes)
    maxC = max(M * N for _, M, N, K, _, _ in shapes)
    A = DeviceArray.from_host(pa.seed_uniform(1, maxA))
    B = DeviceArray.from_host(pa.seed_uniform(2, maxB))
    C = DeviceArray(maxC)
    total_flop, total_ms, rows = 0.0, 0.0, []
    for op, M, N, K, count, acc in shapes:
        lda = K if op != 1 else M
        ldb = N if op != 2 else K
        pa._ffi.check(L.ptmi_gemm_dev(op, A.ptr, lda, B.ptr, ldb, C.ptr, N, M, N, K, 0, None))
        pa._ffi.check(L.ptmi_sync())

        def enqueue():
            for _ in range(reps):
                pa._ffi.check(L.ptmi_gemm_dev(op, A.ptr, lda, B.ptr, ldb, C.ptr, N, M, N, K, acc, stream))

        g = Graph(stream, enqueue)
        g.launch()
        e0, e1 = Event(), Event()
        e0.record(stream)
        for _ in range(3):
            g.launch()
        e1.record(stream)
        ms = e0.elapsed_ms(e1) / (3 * reps)
        g.free()
        flop = 2.0 * M * N * K
        total_flop += flop * count
        total_ms += ms * count
        rows.append({"op": "NN TN NT".split()[op], "M": M, "N": N, "K": K, "count": count, "acc": acc,
                     "us": round(ms * 1e3, 2), "TFLOPs": round(flop / (ms * 1e-3) / 1e12, 2)})
    for a in (A, B, C):
        a.free()
    tflops = total_flop / (total_ms * 1e-3) / 1e12
    out = {"workload": "stories15M training step, T=256, lr=1e-3 (config 5)", "ms_per_step": round(step_ms, 3),
           "losses_first_last": [round(losses[0], 6), round(losses[-1], 6)],
           "losses_steps": "steps 4 and 21 of 21 consecutive SGD steps on one token sequence "
                           "(the first 3 untimed; the timed ms_per_step covers steps 4..21)",
           "gemm_gflop_per_step": round(total_flop / 1e9, 3), "gemm_ms_per_step": round(total_ms, 4),
           "gemm_ms_per_step_basis": "sum over the step's GEMM shapes of isolated graph-replayed launches",
           "gemm_tflops": round(tflops, 2), "gemm_frac_fp32_mfma": round(tflops / MFMA_FP32_PEAK_TFLOPS, 4)}
    # the same GEMMs inside the step: summed kernel durations per step from
    # the committed eager kernel trace (bench.py --train-trace-workload)
    ins, note = committed_in_step()
    out["in_step"] = (None if ins is None else
                      {"gemm_ms": round(ins["gemm_ms"], 4), "kernels_ms": round(ins["kernels_ms"], 4),
                       "gemm_tflops": round(total_flop / ins["gemm_ms"] / 1e9, 2),
                       "gemm_frac_fp32_mfma": round(total_flop / ins["gemm_ms"] / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
                       "basis": f"rocprofv3 kernel trace of {ins['steps']} eager steps "
                                f"({os.path.relpath(TRAIN_PROFILE, ROOT)}, sources {train_sources_hash()})"})
    if note:
        out["in_step_note"] = note
    out["by_shape"] = rows
    return out


def calib_copy(pa, mb=256):
    """One device-to-device copy of known size: the reference point for the
    FETCH_SIZE / WRITE_SIZE counters of the HBM-traffic profiles."""
    from pitorch_amd._hip import DeviceArray, hip
    n = mb * (1 << 20) // 4
    a, b = DeviceArray(n), DeviceArray(n)
    hip().hipMemcpy(b.ptr, a.ptr, n * 4, 3)
    hip().hipDeviceSynchronize()
    a.free()
    b.free()


def pmc_workload(pa, name, positions):
    """Decode positions 0..positions-1 with the step's launches enqueued
    directly (no graph), eight steps per synchronisation, then the copy that
    calibrates FETCH_SIZE / WRITE_SIZE.  The input token of each chunk is
    fixed: the bytes moved do not depend on it."""
    os.environ["PTMI_DECODE_EAGER"] = "1"
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    prompt = pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, cfg[5])
    L = pa.load_ptmi()
    for path in ("1", "0"):                      # the one-kernel step, then the multi-kernel step
        os.environ["PTMI_DECODE_STEP"] = path
        m = pa.Model(blob)
        m.reset_kv()
        for k in range(0, positions, 8):
            m.decode_async(int(prompt[0]), min(8, positions - k))
            m.sync()
        m.close()
    os.environ.pop("PTMI_DECODE_STEP")
    calib_copy(pa)
    print(f"[bench] pmc workload: {positions} positions of {name} on both decode paths, then the calibration copy",
          file=sys.stderr)


def step_stamps(pa, name, at, out=""):
    """The one-kernel decode step's stage timeline (PTMI_DECODE_STEP=1 with
    stage stamps): a greedy decode from position 0; for the step at each
    position in `at`, every workgroup's stamps (the GPU's 100 MHz real-time
    counter) give, per stage and layer: the span, from the last workgroup
    finishing the previous stage to the last finishing this one; the
    release, from that same point to the median workgroup of this stage
    seeing its input (the hand-off); and the median work after the release.
    Medians and maxima are over the layers.  Prints markdown on stdout;
    `out` (a .npz path) also keeps every workgroup's raw stamps per position."""
    import numpy as np
    os.environ["PTMI_DECODE_STEP"] = "1"
    os.environ["PTMI_STEP_STAMPS"] = "1"
    cfg = pa.STORIES[name]
    L = cfg[2]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    prompt = pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, cfg[5])
    m = pa.Model(blob)
    stages = ["qkv", "attention", "wo", "w13", "w2"]
    us = 0.01                                    # one tick = 10 ns
    print("| position | stage | workgroups | span median µs | span max µs | release median µs | release max µs "
          "| work median µs |")
    print("|---:|---|---:|---:|---:|---:|---:|---:|")
    rows = []
    raw = {}
    tok = int(prompt[0])
    for pos in range(max(at) + 1):
        nxt = m.forward_step(tok)
        tok = int(prompt[pos + 1]) if pos + 1 < len(prompt) else nxt
        if pos not in at:
            continue
        st = m.step_stamps().astype(np.int64)
        raw[f"pos{pos}"] = st
        span = {s_: [] for s_ in stages}
        rel = {s_: [] for s_ in stages}
        work = {s_: [] for s_ in stages}
        n_wg = {}
        prev_end = st[:, 0].max()                # the last workgroup's start
        layer_ends = [prev_end]
        for l in range(L):
            for k, s_ in enumerate(stages):
                we, wk = st[:, 1 + 10 * l + 2 * k], st[:, 2 + 10 * l + 2 * k]
                part = (we > 0) & (wk > 0)
                n_wg[s_] = int(part.sum())
                end = wk[part].max()
                span[s_].append((end - prev_end) * us)
                rel[s_].append((np.median(we[part]) - prev_end) * us)
                work[s_].append(np.median((wk - we)[part]) * us)
                prev_end = end
            layer_ends.append(prev_end)
        for s_ in stages:
            print(f"| {pos} | {s_} | {n_wg[s_]} | {np.median(span[s_]):.2f} | {max(span[s_]):.2f} | "
                  f"{np.median(rel[s_]):.2f} | {max(rel[s_]):.2f} | {np.median(work[s_]):.2f} |")
        layer = np.diff(np.array(layer_ends)) * us
        total = (st[st > 0].max() - st[:, 0].min()) * us
        # the step's two ends: workgroup starts, then the classifier (from
        # the last w2 workgroup to the last classifier workgroup) and the
        # final argmax on workgroup 0 (its wait for every candidate, then
        # the end)
        c0 = 1 + 10 * L
        cls_end = st[:, c0 + 1][st[:, c0 + 1] > 0].max()
        rows.append((pos, np.median(layer), layer.max(), total, (st[:, 0].max() - st[:, 0].min()) * us,
                     (cls_end - prev_end) * us, (st[0, c0 + 2] - cls_end) * us, (st[0, c0 + 3] - st[0, c0 + 2]) * us))
    print()
    print("| position | layer median µs | layer max µs | step (first start to last stamp) µs "
          "| workgroup start spread µs | classifier span µs | argmax release µs | argmax work µs |")
    print("|---:|---:|---:|---:|---:|---:|---:|---:|")
    for pos, med, mx, total, spread, cls, arel, awork in rows:
        print(f"| {pos} | {med:.2f} | {mx:.2f} | {total:.2f} | {spread:.2f} | {cls:.2f} | {arel:.2f} | {awork:.2f} |")
    if out:
        np.savez_compressed(out, **raw)
    m.close()


def train_trace_workload(pa, steps):
    """Kernel-trace workload of the training step, no timing: `steps`
    training steps of stories15M at T=256 enqueued eagerly (no graph), each
    waited for (the step returns its loss)."""
    os.environ["PTMI_TRAIN_EAGER"] = "1"
    name, T, lr = "stories15M", 256, 1e-3
    cfg = pa.STORIES[name]
    m = pa.Model(pa.synth_model(cfg, pa.SEED_MODEL[name]), max_T=T)
    tokens = pa.seed_tokens(pa.SEED_TRAIN, T, cfg[5])
    for i in range(steps):
        m.train_step(tokens, lr)
    m.close()
    print(f"[bench] train trace workload: {steps} eager stories15M T=256 steps", file=sys.stderr)


def pmc_gemm(pa, reps):
    """Every training GEMM shape of stories15M at T=256, `reps` launches
    each, enqueued directly (no graph) with one synchronisation per shape:
    the workload of the GEMM counter passes."""
    from pitorch_amd._hip import DeviceArray

    L = pa.load_ptmi()
    shapes = train_gemm_shapes(pa.STORIES["stories15M"], 256)
    A = DeviceArray.from_host(pa.seed_uniform(1, max(M * K for _, M, N, K, _, _ in shapes)))
    B = DeviceArray.from_host(pa.seed_uniform(2, max(K * N for _, M, N, K, _, _ in shapes)))
    C = DeviceArray(max(M * N for _, M, N, K, _, _ in shapes))
    for op, M, N, K, _, acc in shapes:
        lda = K if op != 1 else M
        ldb = N if op != 2 else K
        for _ in range(reps):
            pa._ffi.check(L.ptmi_gemm_dev(op, A.ptr, lda, B.ptr, ldb, C.ptr, N, M, N, K, acc, None))
        pa._ffi.check(L.ptmi_sync())
    for a in (A, B, C):
        a.free()
    print(f"[bench] pmc gemm workload: {len(shapes)} training GEMM shapes x {reps}", file=sys.stderr)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5, help="timed full 1024-position decodes")
    ap.add_argument("--warmup", type=int, default=1, help="untimed full decodes first")
    ap.add_argument("--config", default="stories110M")
    ap.add_argument("--profile-steps", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-train", action="store_true", help="skip the training-GEMM leg")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the standalone matvec sweep (its graph capture does not run under rocprofv3's "
                         "kernel trace on this image: the profiler's host side faults)")
    ap.add_argument("--only-train", action="store_true",
                    help="run only the training leg and print its JSON (for counter profiles), not the bench line")
    ap.add_argument("--pmc-gemm", type=int, default=0, metavar="REPS",
                    help="only enqueue every training GEMM shape REPS times without graphs (workload for "
                         "rocprofv3 --pmc passes), print nothing on stdout")
    ap.add_argument("--pmc-workload", type=int, default=0, metavar="POSITIONS",
                    help="counter-profile workload, no timing: POSITIONS decode steps of the --config model "
                         "enqueued without graphs, 8 at a time (rocprofv3 --pmc faults on its host side with "
                         "thousands of dispatches in flight), then the 256 MiB calibration copy")
    ap.add_argument("--train-trace-workload", type=int, default=0, metavar="STEPS",
                    help="kernel-trace workload, no timing: STEPS eager training steps (no graph launches), "
                         "print nothing on stdout")
    ap.add_argument("--stamps-out", type=str, default="", metavar="NPZ",
                    help="with --step-stamps: also save every workgroup's raw stamps")
    ap.add_argument("--step-stamps", type=str, default="", metavar="POSITIONS",
                    help="print the one-kernel decode step's stage timeline at these comma-separated positions "
                         "(greedy decode of the --config model from position 0), not the bench line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a code path", file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import pitorch_amd as pa

    if args.only_train:
        print(json.dumps(bench_train(pa)), flush=True)
        return
    if args.pmc_gemm:
        pmc_gemm(pa, args.pmc_gemm)
        return
    if args.pmc_workload:
        pmc_workload(pa, args.config, args.pmc_workload)
        return
    if args.train_trace_workload:
        train_trace_workload(pa, args.train_trace_workload)
        return
    if args.step_stamps:
        step_stamps(pa, args.config, sorted(int(p) for p in args.step_stamps.split(",")), args.stamps_out)
        return

    name = args.config
    cfg = pa.STORIES[name]
    S = cfg[6]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    prompt = pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, cfg[5])
    m = pa.Model(blob)
    L = pa.load_ptmi()
    print(f"[bench] {name} model resident ({blob.nbytes / 1e6:.1f} MB)", file=sys.stderr, flush=True)

    # warmup: full decodes (graph replays at every position, steady clocks)
    gen = lambda: m.generate(prompt, S, stop_on_eos=False)
    for _ in range(args.warmup):
        gen()

    # timed: K full decodes of positions 0..S-1, back to back (each one
    # zeroes the KV cache, forces the prompt, then decodes greedily; the
    # host waits once per decode)
    pa._ffi.check(L.ptmi_sync())
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks = gen()
        assert len(toks) == S
    pa._ffi.check(L.ptmi_sync())
    dt = time.perf_counter() - t0
    n_tok = args.steps * S
    tok_s = n_tok / dt
    print(f"[bench] {args.steps} decodes x {S} positions in {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s",
          file=sys.stderr, flush=True)

    # per-kernel durations: eager steps over the same positions, each launch
    # bracketed by HIP events that the command processor stamps at the
    # kernel's own start and end (hipExtLaunchKernelGGL), library stream
    m.reset_kv()
    n_prof = min(args.profile_steps, S)
    rb = role_bytes(cfg, range(n_prof))

    def per_role(model):
        prof = model.profile(int(prompt[0]), n_prof)
        out = {}
        for role, (ms, cnt) in prof.items():
            if cnt == 0:
                continue
            avg_us = ms * 1e3 / cnt
            out[role] = {"avg_us": round(avg_us, 3), "launches": cnt, "total_ms": round(ms, 4),
                         "bytes_per_launch": rb[role], "GBps": round(rb[role] / (avg_us * 1e-6) / 1e9, 1)}
        return out

    breakdown = per_role(m)
    one_kernel = "step" in breakdown
    dominant = max(breakdown, key=lambda r: breakdown[r]["total_ms"])
    dom = breakdown[dominant]
    achieved = dom["GBps"]
    kernel_ms = sum(e["total_ms"] for e in breakdown.values()) / n_prof
    for r, e in breakdown.items():
        print(f"[bench] {r:12s} {json.dumps(e)}", file=sys.stderr, flush=True)
    step_bytes = decode_bytes_per_token(cfg, range(S))
    step_gbs = step_bytes / (dt / n_tok) / 1e9
    m.close()

    # the same decode on the other path (the captured multi-kernel step when
    # the default is the one-kernel step), timed the same way, with its
    # per-kernel breakdown
    os.environ["PTMI_DECODE_STEP"] = "0" if one_kernel else "1"
    m2 = pa.Model(blob)
    os.environ.pop("PTMI_DECODE_STEP")
    gen2 = lambda: m2.generate(prompt, S, stop_on_eos=False)
    for _ in range(args.warmup):
        gen2()
    pa._ffi.check(L.ptmi_sync())
    t0 = time.perf_counter()
    for _ in range(args.steps):
        gen2()
    pa._ffi.check(L.ptmi_sync())
    other = {"path": "multi_kernel" if one_kernel else "one_kernel",
             "tok_s": round(n_tok / (time.perf_counter() - t0), 2)}
    m2.reset_kv()
    other["breakdown"] = per_role(m2)
    m2.close()
    print(f"[bench] other path {json.dumps({k: v for k, v in other.items() if k != 'breakdown'})}",
          file=sys.stderr, flush=True)
    del blob
    sweep = None if args.no_sweep else matvec_sweep(pa)
    for e in sweep or []:
        print(f"[bench] sweep {json.dumps(e)}", file=sys.stderr, flush=True)
    calib_copy(pa)
    train = None if args.no_train else bench_train(pa)
    if train:
        print(f"[bench] train {json.dumps({k: v for k, v in train.items() if k != 'by_shape'})}", file=sys.stderr,
              flush=True)
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    cpu = None if args.no_cpu else cpu_baseline(blob, prompt, S)
    del blob
    cpu_more = None if args.no_cpu else cpu_extra()
    # measured HBM bytes per launch of the dominant kernel (fetch + write,
    # counter-calibrated), from the committed passes over all S positions,
    # when they were measured on this build's decode sources
    if n_prof == S:
        traffic, traffic_note = committed_traffic(dominant, name)
    else:
        traffic, traffic_note = None, f"traffic was measured over positions 0..{S - 1}, this run profiles {n_prof}"

    line = {
        "metric": "decode tok/s + matvec HBM GB/s (% peak), stories110M-shape fp32, 1 GPU",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init N(0,0.02) weights, seeded prompt ids)",
        "config": {"workload": f"{name}-shaped greedy decode, "
                               + ("one kernel per token" if one_kernel else "62 kernels per token")
                               + ", hipGraphs of 8 tokens", "model_shape": list(cfg),
                   "step": f"one full greedy decode of positions 0..{S - 1} (pt_generate over ids)",
                   "positions": f"0..{S - 1}", "tokens_timed": n_tok, "batch": 1},
        "roofline": {"bound": "hbm", "kernel": f"decode[{dominant}]", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_sources": decode_sources_hash(),
                     **({"traffic_note": traffic_note} if traffic_note else {}),
                     "bytes_per_launch": dom["bytes_per_launch"], "avg_us": dom["avg_us"]},
        "step_roofline": {"bytes_per_token": int(step_bytes), "achieved_GBps": round(step_gbs, 1),
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4), "kernel_ms_per_token": round(kernel_ms, 4)},
        "matvec_sweep": sweep,
        "cpu_baseline": cpu,
        "cpu_extra": cpu_more,
        "breakdown": breakdown,
        "other_path": other,
        "train": train,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
