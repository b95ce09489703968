#!/usr/bin/env python3
"""bench.py -- headline benchmark of the quantized-weight matrix path on one
MI355X.

Step (the timed unit): one decode step's worth of quantised linears of
Qwen2.5-7B at 1 activation row (the headline configuration): 28 layers x (q 3584x3584,
k/v 512x3584, o 3584x3584, gate/up 18944x3584, down 3584x18944) in int4
(group 128, bf16 scale, u8 zero point) plus the int8 lm_head 152064x3584,
weights seeded ~N(0, 0.02) -> bf16 -> quantised on the device (bit-exact to
src/quant.cpp), activations fp32 ~N(0, 1).  The step is issued the way a
decode engine issues it -- one call per distinct input (attention input:
q|k|v in one call; attention context: o; MLP input: gate|up in one call;
MLP hidden: down; final norm: lm_head) -- and captured in one HIP graph, as
the reference's engine captures its step (kernels/batch_gpu.cu:255-269).

value = packed weight bytes + activation bytes read + output bytes written,
per step, / time per step (GB/s).  All inputs are resident in HBM before the
timed region; the 7B set is ~4 GB, far beyond the 256 MB MALL, so each step
streams the weights from HBM.

Also reported (measured after the timed region, outside it):
  roofline   the GEMV kernel alone (int4, 1 row): its 112 launches (q|k|v,
             o, gate|up, down of 28 layers) timed with HIP events on their
             stream, grouped by matrix shape and run back to back; traffic
             from profiles/gemv_int4_7b_m1_traffic.json (rocprofv3 counters);
  cpu_baseline  the reference CPU path (src/forward.cpp linear over dequant(),
             restated in oracle/iq_oracle.c) on a bounded sample, 1 thread;
  detail     per-shape GB/s of the 1-row launches, int4 at 16 rows (and at
             2, 4, 8 and 32 rows: 7b_int4_rows_sweep), the decode
             step chained as the engine runs it (norms, attention at position
             0, SwiGLU, residuals fused into the GEMV stages), the int8 set
             at 1 and 16 rows, the prefill GEMM (config 5), on-device
             quantize, configs 1-3.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "dequant-GEMV GB/s & % HBM peak, 7B int4/int8 at 1/16 rows; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

H7, I7, NH7, KV7, V7, L7 = 3584, 18944, 28, 4, 152064, 28
H15, I15, L15 = 1536, 8960, 28


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_shapes(H, I, q_out, kv_out):
    # (name, out, in, activation slot)
    return [("q", q_out, H, "attn"), ("k", kv_out, H, "attn"), ("v", kv_out, H, "attn"),
            ("o", H, q_out, "ctx"), ("gate", I, H, "mlp"), ("up", I, H, "mlp"), ("down", H, I, "hid")]


class Model:
    """Seeded quantised linears of one model, resident on the device."""

    def __init__(self, torch, ops, kind, H, I, q_out, kv_out, layers, head=None, seed=0):
        self.torch, self.ops = torch, ops
        self.kind = kind
        self.H, self.I = H, I
        self.shapes = layer_shapes(H, I, q_out, kv_out)
        self.layers = []
        gen = torch.Generator(device="cuda")
        for li in range(layers):
            mats = {}
            for j, (name, out, inn, slot) in enumerate(self.shapes):
                gen.manual_seed(seed * 1000003 + li * 16 + j)
                mats[name] = quantize_seeded(torch, ops, kind, out, inn, gen)
            self.layers.append(mats)
        self.head = None
        if head is not None:
            hk, V = head
            gen.manual_seed(seed * 1000003 + 999)
            self.head = quantize_seeded(torch, ops, hk, V, H, gen)

    def weight_bytes(self):
        n = sum(W.nbytes() for L in self.layers for W in L.values())
        return n + (self.head.nbytes() if self.head is not None else 0)


def quantize_seeded(torch, ops, kind, out, inn, gen):
    w = (torch.randn(out, inn, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    W = ops.quantize(w.view(torch.int16), kind)
    del w
    return W


class Step:
    """One decode step over a Model at M rows: the op list and its bytes."""

    def __init__(self, torch, ops, model, M, seed=1):
        self.torch, self.ops, self.model, self.M = torch, ops, model, M
        g = torch.Generator(device="cuda").manual_seed(seed)
        H, I = model.H, model.I
        self.x = {"attn": torch.randn(M, H, generator=g, device="cuda"),
                  "ctx": torch.randn(M, model.layers[0]["o"].cols, generator=g, device="cuda"),
                  "mlp": torch.randn(M, H, generator=g, device="cuda"),
                  "hid": torch.randn(M, I, generator=g, device="cuda"),
                  "head": torch.randn(M, H, generator=g, device="cuda")}
        self.y = {name: torch.empty(M, out, device="cuda") for name, out, _, _ in model.shapes}
        if model.head is not None:
            self.y["head"] = torch.empty(M, model.head.rows, device="cuda")
        # op list: (activation slot, [W...], [yname...]); matrices that share
        # an activation (q|k|v, gate|up) go in one call.
        self.ops_list = []
        for L in model.layers:
            last = None
            for name, out, inn, slot in model.shapes:
                if slot != last:
                    self.ops_list.append((slot, [], []))
                    last = slot
                self.ops_list[-1][1].append(L[name])
                self.ops_list[-1][2].append(name)
        if model.head is not None:
            self.ops_list.append(("head", [model.head], ["head"]))
        self.bytes = 0
        for _, Ws, _ in self.ops_list:
            for W in Ws:
                self.bytes += W.nbytes() + 4 * M * W.rows
            self.bytes += 4 * M * Ws[0].cols

    def run(self):
        ops, M = self.ops, self.M
        for slot, Ws, ynames in self.ops_list:
            self.launch(slot, Ws, ynames)

    def launch(self, slot, Ws, ynames):
        x = self.x[slot]
        self.ops.gemv_multi(x, Ws, None, self.M, x.shape[1], [self.y[n] for n in ynames])

    def capture(self):
        torch = self.torch
        self.run()  # eager warm-up: workspace and code objects resident
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=capture_stream(torch)):
            self.run()
        torch.cuda.synchronize()
        return g


_CAPTURE = None


def capture_stream(torch):
    """The one stream every graph here is captured on, its library
    workspace reserved first (a capturing stream cannot allocate one)."""
    global _CAPTURE
    if _CAPTURE is None:
        from infer_amd import ops as iq_ops
        _CAPTURE = torch.cuda.Stream()
        iq_ops.init(0, _CAPTURE)
    return _CAPTURE


def time_graph(torch, g, steps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) / steps


def kernel_roofline(torch, step, only_kind=None):
    """Average GEMV launch duration from HIP events on the launch stream
    (torch's current stream, which the ctypes calls pass down).  The step's
    GEMV launches are grouped by their place in a layer (q|k|v, o, gate|up,
    down); each group's launches (one per layer, each on its own weights) run
    back to back between two events.  A device-side sleep queued first lets
    the host enqueue everything before the GPU reaches it, so the events
    bracket kernels and not host launch latency."""
    groups = {}
    for op in step.ops_list:
        Ws = op[1]
        key = tuple(W.rows for W in Ws) + (Ws[0].cols, Ws[0].kind)
        groups.setdefault(key, []).append(op)
    M = step.M
    timing = []
    torch.cuda._sleep(int(2.4e9 * 0.05))
    for key, gops in groups.items():
        if only_kind is not None and key[-1] != only_kind:
            continue
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for op in gops:
            step.launch(*op)
        e1.record()
        nb = sum(sum(W.nbytes() + 4 * M * W.rows for W in Ws) + 4 * M * Ws[0].cols
                 for _, Ws, _ in gops)
        timing.append((nb, len(gops), e0, e1))
    torch.cuda.synchronize()
    tot_b, tot_ms, n = 0, 0.0, 0
    per_shape = {}
    for (nb, cnt, e0, e1), key in zip(timing, [k for k in groups if only_kind is None or k[-1] == only_kind]):
        ms = e0.elapsed_time(e1)
        tot_b += nb
        tot_ms += ms
        n += cnt
        name = "|".join(str(r) for r in key[:-2]) + f"x{key[-2]}"
        per_shape[name] = {"launches": cnt, "avg_us": round(ms * 1e3 / cnt, 2),
                           "bytes_per_launch": int(nb / cnt), "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                           "frac_hbm_peak": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return tot_b, tot_ms, n, per_shape


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), for the baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, model, seconds=10.0, threads=1):
    """oracle/iq_oracle.c iqo_linear_q_f32 (= src/forward.cpp:35-47 over
    dequant(), one thread) on layer matrices of the same model, until about
    `seconds` of CPU work; returns (GB/s of packed weights, sample text).
    threads > 1: each matrix's output rows split over that many host threads
    (the C routine runs without the GIL; every output is computed exactly as
    with one thread)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import oracle as O
    rng = np.random.default_rng(0)
    done_b, t_tot, n = 0, 0.0, 0
    names = []
    pool = ThreadPoolExecutor(threads) if threads > 1 else None
    for li, L in enumerate(model.layers):
        for name, out, inn, slot in model.shapes:
            W = L[name]
            q = W.q.cpu().numpy().reshape(W.rows, -1)
            s = W.scales.cpu().numpy().view(np.uint16).reshape(W.rows, W.groups)
            z = W.zeros.cpu().numpy().reshape(W.rows, W.groups) if W.zeros is not None else None
            x = rng.standard_normal((1, W.cols), dtype=np.float32)
            t0 = time.perf_counter()
            if pool is None:
                O.linear_q_f32(x, q, s, z, int(W.kind), None, W.rows)
            else:
                cuts = [W.rows * i // threads for i in range(threads + 1)]
                jobs = [pool.submit(O.linear_q_f32, x, q[a:b], s[a:b], None if z is None else z[a:b],
                                    int(W.kind), None, b - a) for a, b in zip(cuts[:-1], cuts[1:]) if b > a]
                for j in jobs:
                    j.result()
            t_tot += time.perf_counter() - t0
            done_b += W.nbytes()
            n += 1
            names.append(f"L{li}.{name}")
            if t_tot >= seconds:
                break
        if t_tot >= seconds:
            break
    return done_b / t_tot / 1e9, f"{n} matrices ({names[0]}..{names[-1]}), {done_b / 1e6:.0f} MB packed, {t_tot:.1f} s"


def cpu_quantize_rate():
    """oracle iqo_quantize (src/quant.cpp:34-84 restated, one thread) on a
    3584 x 3584 bf16 matrix, int8 and int4: GB/s of bf16 read."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(1)
    w = O.seeded_bf16(rng, (3584, 3584), 0.02)
    out = {}
    for kind, kn in ((0, "int8"), (1, "int4")):
        t0 = time.perf_counter()
        O.quantize(w, kind)
        dt = time.perf_counter() - t0
        out[kn] = {"ms": round(dt * 1e3, 1), "GBps": round(w.nbytes / dt / 1e9, 3)}
    out["sample"] = "3584 x 3584 bf16, 1 thread"
    return out


def hbm_copy_rate(torch, reps=20):
    """A plain device copy of 2 GiB (torch copy_): bytes read + written per
    second, the measured HBM ceiling beside the nominal 8 TB/s."""
    a = torch.empty(512 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del a, b
    torch.cuda.empty_cache()
    return round(2 * (2 << 30) / (ms * 1e-3) / 1e9, 1)


def bench_gemm(torch, ops, kind, T, N, K, reps=10, seed=5, fp32x=False):
    """Prefill GEMM at config 5: bf16 activations (iq_gemm_bf16x), or fp32
    activations through the reference-compatible launch_gemm_tiled_q (one
    preparation launch into fp16 hi + lo operands, then two MFMAs per
    product; the timing includes the preparation)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = quantize_seeded(torch, ops, kind, N, K, g)
    xf = torch.randn(T, K, generator=g, device="cuda")
    x = xf.to(torch.bfloat16)
    y = torch.empty(T, N, device="cuda")

    def run():
        if fp32x:
            ops.launch_gemm_tiled_q(xf, W, None, T, K, N, y)
        else:
            ops.launch_gemm_bf16x(x.view(torch.int16), W, None, T, K, N, y)
    for _ in range(2):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    return ms, 2.0 * T * N * K / (ms * 1e-3) / 1e12


def bench_quantize_model(torch, ops):
    """Config 5b: the 7B model's 198 matrices (bf16 ~N(0, 0.02), seeded)
    quantised by iq_quantize one after another, int8 and int4; returns per
    kind the total time, bf16 GB/s read and bytes read + written per
    second."""
    shapes = []
    for _ in range(L7):
        shapes += [(NH7 * 128, H7), (KV7 * 128, H7), (KV7 * 128, H7), (H7, NH7 * 128), (I7, H7), (I7, H7), (H7, I7)]
    shapes += [(V7, H7), (V7, H7)]
    g = torch.Generator(device="cuda").manual_seed(11)
    ws = [(torch.randn(r, c, generator=g, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
          for r, c in shapes]
    params = sum(r * c for r, c in shapes)
    res = {"matrices": len(shapes), "params": params}
    for kind, kn in ((0, "int8"), (1, "int4")):
        outs = [ops.alloc_quant(kind, r, c) for r, c in shapes]
        for w, o in zip(ws[:8], outs[:8]):
            ops.quantize(w, kind, out=o)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for w, o in zip(ws, outs):
            ops.quantize(w, kind, out=o)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        written = sum(o.nbytes() for o in outs)
        res[kn] = {"ms": round(ms, 3), "bf16_read_GBps": round(2 * params / (ms * 1e-3) / 1e9, 1),
                   "GBps": round((2 * params + written) / (ms * 1e-3) / 1e9, 1),
                   "frac_hbm_peak": round((2 * params + written) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        # the same 198 launches captured in one graph and replayed: the
        # device's rate when the launches are enqueued back to back (the
        # eager loop above waits on Python for the small k / v matrices,
        # whose kernels take ~1.5 us)
        cs = capture_stream(torch)
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=cs):
            for w, o in zip(ws, outs):
                ops.quantize(w, kind, out=o, stream=cs)
        gr.replay()
        torch.cuda.synchronize()
        reps = 3
        e0.record()
        for _ in range(reps):
            gr.replay()
        e1.record()
        torch.cuda.synchronize()
        gms = e0.elapsed_time(e1) / reps
        res[kn]["graph"] = {"ms": round(gms, 3), "GBps": round((2 * params + written) / (gms * 1e-3) / 1e9, 1),
                            "frac_hbm_peak": round((2 * params + written) / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del gr
        del outs
    del ws
    return res


def bench_gemv_single(torch, ops, kind, N, K, M, copies, reps=200, seed=11):
    """One matrix shape rotated over `copies` distinct weight copies (beyond the
    MALL), iq_gemv per call, captured in a graph of `copies` launches."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    Ws = [quantize_seeded(torch, ops, kind, N, K, g) for _ in range(copies)]
    x = torch.randn(M, K, generator=g, device="cuda")
    y = torch.empty(M, N, device="cuda")

    def run():
        for W in Ws:
            ops.launch_gemv_batched_q(x, W, None, M, K, N, y)
    run()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=capture_stream(torch)):
        run()
    reps_g = max(1, reps // copies)
    ms_step, _ = time_graph(torch, gr, reps_g, 2)
    per_ms = ms_step / copies
    nb = Ws[0].nbytes() + 4 * M * K + 4 * M * N
    del Ws, gr
    torch.cuda.empty_cache()
    return per_ms * 1e3, nb / (per_ms * 1e-3) / 1e9


def bench_decode_chain(torch, ops, model, steps, warmup, rows=1):
    """The quantised decode step as the reference's engine chains it
    (kernels/batch_gpu.cu:186-215), one token at position 0: embedding
    gather, then per layer RMSNorm -> q|k|v, single-key attention -> o +
    residual, RMSNorm -> gate|up with the SwiGLU epilogue, down + residual,
    and the final RMSNorm -> lm_head, every stage reading the previous
    stage's output (infer_amd/chain.py; one launch per stage, captured in a
    HIP graph).  Same weights as the headline step; random bf16 norm
    weights and q/k/v biases; the int8 lm_head doubles as the embedding
    table.  GB/s counts the packed weights read per step."""
    from infer_amd import chain as C
    g = torch.Generator(device="cuda").manual_seed(21)
    nb = lambda n: (torch.rand(n, generator=g, device="cuda") * 0.8 + 0.6).to(torch.bfloat16).view(torch.int16)
    cfg = dict(hidden=H7, inter=I7, heads=NH7, kv_heads=KV7, head_dim=128, vocab=V7, layers=len(model.layers),
               eps=1e-6)
    layers = []
    for L in model.layers:
        d = dict(L)
        d["input_ln"], d["post_ln"] = nb(H7), nb(H7)
        d["q_b"], d["k_b"], d["v_b"] = nb(NH7 * 128), nb(KV7 * 128), nb(KV7 * 128)
        layers.append(d)
    spec = dict(cfg=cfg, layers=layers, embed=model.head, head=model.head, final_norm=nb(H7))
    step = C.DecodeStep(spec, rows=rows)
    step.step([1234 + 7 * b for b in range(rows)])
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=capture_stream(torch)):
        step.step()
    ms, _ = time_graph(torch, gr, steps, warmup)
    wb = step.weight_bytes()
    out = {"us_per_step": round(ms * 1e3, 1), "GBps": round(wb / (ms * 1e-3) / 1e9, 1),
           "frac_hbm_peak": round(wb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "rows": rows,
           "launches": (len(step.chain.stages) if rows == 1 else 2 * len(step.chain.stages)) + 1,
           "weight_bytes": int(wb),
           # the quantised linears of one decode step per second (attention
           # over a KV cache, sampling and the host are not in it; the
           # reference's 7B int4 end to end: 126 tok/s on an RTX 5070 Ti,
           # README.md:57)
           "steps_per_s_linears_only": round(1e3 / ms, 1),
           "tokens_per_s_linears_only": round(rows * 1e3 / ms, 1),
           "logits_finite": bool(torch.isfinite(step.logits).all().item())}
    del gr, step
    return out


def profile_workload(torch, ops):
    """Fixed short workload for `rocprofv3 --pmc` runs: 4 layers of the 7B
    int4 set at 1 row (q|k|v, o, gate|up, down launches as in the step), then
    a plain 256 MiB device copy (3 times) whose FETCH_SIZE / WRITE_SIZE per
    dispatch calibrate the counters (known bytes read and written)."""
    m4 = Model(torch, ops, 1, H7, I7, NH7 * 128, KV7 * 128, 4, head=None, seed=7)
    st = Step(torch, ops, m4, 1)
    for _ in range(3):
        st.run()
    torch.cuda.synchronize()
    a = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def profile_gemm_workload(torch, ops):
    """Fixed short workload for `rocprofv3 --pmc` runs of the prefill GEMM
    (config 5, T = 1024): int8 and int4 gate/up 18944x3584 and down
    3584x18944, bf16 then fp32 activations, each launched 2 + 3 times by
    bench_gemm."""
    for fp32x in (False, True):
        for kind in (0, 1):
            for N, K in ((I7, H7), (H7, I7)):
                bench_gemm(torch, ops, kind, 1024, N, K, reps=3, fp32x=fp32x)
    torch.cuda.synchronize()


def profile_rows_workload(torch, ops, M):
    """Fixed short workload for `rocprofv3` runs of the M-row decode set: 4
    layers of the 7B int4 set at M activation rows (the launches of the timed
    step at that width, preparation launches included), run 3 times."""
    m4 = Model(torch, ops, 1, H7, I7, NH7 * 128, KV7 * 128, 4, head=None, seed=7)
    st = Step(torch, ops, m4, M)
    for _ in range(3):
        st.run()
    torch.cuda.synchronize()


def profile_quantize_workload(torch, ops):
    """Fixed short workload for `rocprofv3 --pmc` runs of the on-device
    quantiser: 18944 x 3584 bf16 -> int8 and int4, 3 launches each."""
    gq = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn(I7, H7, generator=gq, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
    for kind in (0, 1):
        out = ops.alloc_quant(kind, I7, H7)
        for _ in range(3):
            ops.quantize(w, kind, out=out)
    torch.cuda.synchronize()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline only (no detail / CPU baseline)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile", action="store_true",
                    help="short fixed workload for rocprofv3 counter runs (prints nothing)")
    ap.add_argument("--profile-gemm", action="store_true",
                    help="short fixed prefill-GEMM workload for rocprofv3 counter runs (prints nothing)")
    ap.add_argument("--profile-quantize", action="store_true",
                    help="short fixed quantize workload for rocprofv3 counter runs (prints nothing)")
    ap.add_argument("--profile-rows", type=int, default=0,
                    help="short fixed M-row decode-set workload for rocprofv3 runs (prints nothing)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the quantized-weight path runs on one GPU here (output rows would split across GPUs).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from infer_amd import ops
    ops.init(0)
    if args.profile:
        profile_workload(torch, ops)
        return
    if args.profile_gemm:
        profile_gemm_workload(torch, ops)
        return
    if args.profile_quantize:
        profile_quantize_workload(torch, ops)
        return
    if args.profile_rows:
        profile_rows_workload(torch, ops, args.profile_rows)
        return
    t_setup = time.perf_counter()

    # ---- headline: 7B int4 set + int8 lm_head, 1 row
    m4 = Model(torch, ops, 1, H7, I7, NH7 * 128, KV7 * 128, L7, head=(0, V7), seed=7)
    torch.cuda.synchronize()
    log(f"setup int4 7B: {m4.weight_bytes() / 1e9:.3f} GB packed in {time.perf_counter() - t_setup:.1f} s")
    st = Step(torch, ops, m4, 1)
    g = st.capture()
    ms_wall, ms_ev = time_graph(torch, g, args.steps, args.warmup)
    step_bytes = st.bytes
    value = step_bytes / (ms_wall * 1e-3) / 1e9
    log(f"int4 M=1: {ms_wall * 1e3:.1f} us/step wall, {ms_ev * 1e3:.1f} us events, {value:.0f} GB/s")
    # per-replay spread (after the timed region): 50 replays, each between
    # its own pair of events
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(50)]
    for a, b in evs:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    step_stats = {"replays": len(per), "median_us": round(per[len(per) // 2], 1), "min_us": round(per[0], 1),
                  "max_us": round(per[-1], 1)}

    # roofline of the dominant kernel (int4 GEMV, 1 row)
    rb, rms, rn, per_shape = kernel_roofline(torch, st, only_kind=1)
    achieved = rb / (rms * 1e-3) / 1e9
    traffic = None
    prof = os.path.join(ROOT, "profiles", "gemv_int4_7b_m1_traffic.json")
    if os.path.exists(prof):
        try:
            traffic = json.load(open(prof)).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "gemv1_kernel (int4, 1 row): the 112 launches of the 28 layers (q|k|v, o, gate|up, down)",
                "launches": rn, "avg_launch_us": round(rms * 1e3 / max(rn, 1), 3),
                "algorithmic_bytes_per_launch": int(rb / max(rn, 1))}
    del g

    detail = {"7b_int4_m1_step_spread": step_stats, "7b_int4_m1_gemv_per_shape": per_shape}
    cpu = None
    if not args.quick:
        st16 = Step(torch, ops, m4, 16)
        g16 = st16.capture()
        ms16, _ = time_graph(torch, g16, args.steps, args.warmup)
        detail["7b_int4_m16"] = {"us_per_step": round(ms16 * 1e3, 1),
                                 "GBps": round(st16.bytes / (ms16 * 1e-3) / 1e9, 1),
                                 "ratio_vs_m1": round(ms16 / ms_wall, 3)}
        del g16, st16
        # the same step at the other batch widths of the reference's decode
        # (GpuBatch::kMaxRows = 32): time and ratio to the 1-row step
        sweep = {}
        for M in (2, 4, 8, 32):
            stm = Step(torch, ops, m4, M)
            gm = stm.capture()
            msm, _ = time_graph(torch, gm, args.steps, args.warmup)
            sweep[str(M)] = {"us_per_step": round(msm * 1e3, 1), "ratio_vs_m1": round(msm / ms_wall, 3)}
            del gm, stm
        detail["7b_int4_rows_sweep"] = sweep
        detail["7b_int4_decode_chain_m1"] = bench_decode_chain(torch, ops, m4, args.steps, args.warmup)
        # the chained step at B sequences (B-row stages), beside the bare
        # linear set at the same widths
        for B in (2, 4, 16, 32):
            dc = bench_decode_chain(torch, ops, m4, args.steps, args.warmup, rows=B)
            dc["ratio_vs_chain_m1"] = round(dc["us_per_step"] / detail["7b_int4_decode_chain_m1"]["us_per_step"], 3)
            detail[f"7b_int4_decode_chain_m{B}"] = dc
        cpu_gbs, cpu_sample = cpu_baseline(torch, m4, args.cpu_seconds)
        cpu = {"value": round(cpu_gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": "oracle iqo_linear_q_f32 (src/forward.cpp:35-47 over dequant(), scalar fp32, "
                         "1 thread) on the 7B int4 layer matrices at 1 row: " + cpu_sample + "; host CPU: " + cpu_model()}
        # the same port over the host's cores (at most 16, the box's share)
        nth = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))
        cpu_all, cpu_all_sample = cpu_baseline(torch, m4, args.cpu_seconds / 2, threads=nth)
        detail["cpu_baseline_all_cores"] = {"value": round(cpu_all, 4), "unit": "GB/s", "cores": nth,
                                            "kind": "port", "sample": cpu_all_sample}
        # CPU quantize (the oracle's restatement of src/quant.cpp:34-84), one thread
        detail["cpu_quantize"] = cpu_quantize_rate()
        del m4, st
        torch.cuda.empty_cache()

        # int8 set
        t0 = time.perf_counter()
        m8 = Model(torch, ops, 0, H7, I7, NH7 * 128, KV7 * 128, L7, head=(0, V7), seed=8)
        torch.cuda.synchronize()
        tq = time.perf_counter() - t0
        for M in (1, 16):
            s8 = Step(torch, ops, m8, M)
            g8 = s8.capture()
            ms8, _ = time_graph(torch, g8, args.steps, args.warmup)
            detail[f"7b_int8_m{M}"] = {"us_per_step": round(ms8 * 1e3, 1),
                                       "GBps": round(s8.bytes / (ms8 * 1e-3) / 1e9, 1)}
            del g8, s8
        detail["7b_int8_setup_s"] = round(tq, 2)
        del m8
        torch.cuda.empty_cache()

        # on-device quantize+pack throughput (gate/up shape, int8 and int4),
        # rotated over 4 distinct weight / output buffers (~0.8 GB, past the
        # 256 MB MALL: one matrix requantised in place is partly served from
        # it, 35 against 44 us for int8)
        gq = torch.Generator(device="cuda").manual_seed(3)
        wr = [(torch.randn(I7, H7, generator=gq, device="cuda") * 0.02).to(torch.bfloat16).view(torch.int16)
              for _ in range(4)]
        for kind, kn in ((0, "int8"), (1, "int4")):
            outs = [ops.alloc_quant(kind, I7, H7) for _ in wr]
            for w, out in zip(wr, outs):
                ops.quantize(w, kind, out=out)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(3):
                for w, out in zip(wr, outs):
                    ops.quantize(w, kind, out=out)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 12
            nb = 2 * I7 * H7 + outs[0].nbytes()
            detail[f"quantize_{kn}_18944x3584"] = {"us": round(ms * 1e3, 1), "GBps": round(nb / (ms * 1e-3) / 1e9, 1)}
            del outs
        del wr
        # config 5b: every matrix of the 7B model (28 layers x q,k,v,o,gate,up,
        # down, the embedding and the lm_head: 7.6 G parameters) quantised on
        # the device back to back, inputs resident (distinct buffers, far past
        # the MALL); tools/quantize.cpp's loop runs this on the CPU
        detail["quantize_7b_all"] = bench_quantize_model(torch, ops)
        torch.cuda.empty_cache()
        # prefill GEMM (config 5), int8, bf16 activations, T = 1024
        for (N, K, nm) in ((I7, H7, "gate_up"), (H7, I7, "down")):
            for kind, kn in ((0, "int8"), (1, "int4")):
                ms, tf = bench_gemm(torch, ops, kind, 1024, N, K)
                detail[f"prefill_{kn}_{nm}_1024"] = {"us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1),
                                                     "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
            ms, tf = bench_gemm(torch, ops, 0, 1024, N, K, fp32x=True)
            detail[f"prefill_int8_{nm}_1024_fp32x"] = {"us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1),
                                                       "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
        # the reference's prefill chunks (32 < T <= 256), fp32 activations
        # (launch_gemm_tiled_q), int8: us and weight GB/s
        chunk = {}
        for T in (64, 256):
            for (N, K, nm) in ((I7, H7, "gate"), (H7, I7, "down")):
                ms, tf = bench_gemm(torch, ops, 0, T, N, K, fp32x=True)
                chunk[f"T{T}_{nm}"] = {"us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1),
                                       "weights_GBps": round(N * K / (ms * 1e-3) / 1e9, 1)}
        detail["prefill_chunks_int8_fp32x"] = chunk
        # config 1: int8 8960x1536, 1 row, rotated over 64 copies
        us, gbs = bench_gemv_single(torch, ops, 0, I15, H15, 1, copies=64)
        detail["cfg1_int8_8960x1536_m1"] = {"us": round(us, 2), "GBps": round(gbs, 1)}
        detail["hbm_copy_2GiB_GBps"] = hbm_copy_rate(torch)
        # config 2: 1.5B int4 layer set x 28, 1 row
        m15 = Model(torch, ops, 1, H15, I15, 12 * 128, 2 * 128, L15, seed=15)
        s15 = Step(torch, ops, m15, 1)
        g15 = s15.capture()
        ms15, _ = time_graph(torch, g15, args.steps, args.warmup)
        detail["cfg2_1.5b_int4_28layers_m1"] = {"us_per_layer_set": round(ms15 * 1e3 / L15, 2),
                                                "us_total": round(ms15 * 1e3, 1),
                                                "GBps": round(s15.bytes / (ms15 * 1e-3) / 1e9, 1)}
        del g15, s15, m15
        torch.cuda.empty_cache()
        # config 3: M sweep on the 1.5B MLP shapes
        sweep = {}
        for kind, kn in ((0, "int8"), (1, "int4")):
            for (N, K, nm) in ((I15, H15, "gate"), (H15, I15, "down")):
                base = None
                row = {}
                for M in (1, 2, 4, 5, 8, 12, 16, 32):
                    us, gbs = bench_gemv_single(torch, ops, kind, N, K, M, copies=32, reps=128)
                    base = base or us
                    row[str(M)] = {"us": round(us, 2), "GBps": round(gbs, 1), "x_m1": round(us / base, 3)}
                sweep[f"{kn}_{nm}_{N}x{K}"] = row
        detail["cfg3_sweep"] = sweep

    rec = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 (int8 lm_head) weights x fp32 activations as per-128-column-group 31-bit fixed point (four byte limbs, rounding <= 2^-31 of the group max): exact int32 MFMA sums, fp32 accumulation",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-7B decode linear set, int4 group-128 (bf16 scale, u8 zero) x 28 layers "
                        "(q,k,v,o,gate,up,down) + int8 lm_head 152064x3584, 1 activation row, HIP graph",
            "rows": 1,
            "bytes_per_step": int(step_bytes),
            "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(rec), flush=True)

if __name__ == "__main__":
    main()
