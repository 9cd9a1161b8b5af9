#!/usr/bin/env python3
"""Benchmark of the MoE layer of Qwen3.6-35B-A3B on one MI355X (synthetic GGUF Q4_K/Q6_K weights).

Workload of the headline number: decode at batch 1 through 40 stacked layers of the full shape (hidden 2048,
256 experts of width 512, top-8, shared expert of width 512; gate/up Q4_K, down Q6_K, fp32 router), all 40
layers' experts resident in HBM (21 GB), a different input vector per layer and step so the routed experts
change (and the 256 MB Infinity Cache cannot serve repeats). One step = one token through the 40 layers, captured
once as a HIP graph per input set and replayed.
  value = microseconds per token per layer (lower is better); hbm_gbps = algorithmic bytes / that time.
Also reported (same JSON line): batched decode at 64 tokens with Zipf(1.1)-shaped routing, and a 4096-token
prefill chunk, each through the 40 layers; the per-stage kernel times of the layer (HIP events, live); the rate
of loading a synthetic GGUF file's experts into HBM (gguf.loader); and the CPU oracle (numpy dequantize + fp32
matmul) timed on a bounded sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import contextlib
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "willow-v2_amd"))
sys.path.insert(0, ROOT)

HIDDEN, INTER, EXPERTS, TOP_K, LAYERS = 2048, 512, 256, 8, 40
Q4K_ROW = HIDDEN // 256 * 144       # 1152 B: a gate/up row
Q6K_ROW = INTER // 256 * 210        # 420 B: a down row
GATE_UP_BYTES = 2 * INTER * Q4K_ROW  # 1,179,648 B per expert
DOWN_BYTES = HIDDEN * Q6K_ROW        # 860,160 B per expert
EXPERT_BYTES = GATE_UP_BYTES + DOWN_BYTES
ROUTER_BYTES = EXPERTS * HIDDEN * 4
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "MoE layer µs/token + achieved HBM GB/s (decode b=1,64); prefill tok/s, MFMA %"


def new_workspace(nbytes, device):
    from gguf.hip.moe import new_workspace as make
    return make(nbytes, device)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gen_q4k(torch, n, gen):
    b = torch.randint(0, 256, (n, 144), dtype=torch.uint8, device="cuda", generator=gen)
    for off in (0, 2):
        d = (torch.randn(n, device="cuda", generator=gen).abs() * 0.01).half()
        b[:, off:off + 2] = d.view(torch.uint8).view(n, 2)
    return b


def gen_q6k(torch, n, gen):
    b = torch.randint(0, 256, (n, 210), dtype=torch.uint8, device="cuda", generator=gen)
    sc = torch.randint(-32, 32, (n, 16), dtype=torch.int8, device="cuda", generator=gen)
    b[:, 192:208] = sc.view(torch.uint8)
    d = (torch.randn(n, device="cuda", generator=gen).abs() * 0.01).half()
    b[:, 208:210] = d.view(torch.uint8).view(n, 2)
    return b


def build_layers(torch, hip, n_layers, zipf=False, seed=1):
    """n_layers independent full-shape layers, generated on the GPU with the same recipes as gguf.synth (the
    bytes differ from the numpy generator's; the distributions are the same)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        gate_up = gen_q4k(torch, EXPERTS * 2 * INTER * (HIDDEN // 256), gen).view(EXPERTS, -1)
        down = gen_q6k(torch, EXPERTS * HIDDEN * (INTER // 256), gen).view(EXPERTS, -1)
        router = torch.randn(EXPERTS, HIDDEN, device="cuda", generator=gen) * 0.02
        sgu = gen_q4k(torch, 2 * INTER * (HIDDEN // 256), gen).view(-1)
        sdn = gen_q6k(torch, HIDDEN * (INTER // 256), gen).view(-1)
        sgate = torch.randn(HIDDEN, device="cuda", generator=gen) * 0.02
        bias = None
        if zipf:
            perm = torch.randperm(EXPERTS, device="cuda", generator=gen)
            bias = torch.empty(EXPERTS, device="cuda")
            bias[perm] = -1.1 * torch.log(torch.arange(1, EXPERTS + 1, device="cuda", dtype=torch.float32))
        layers.append(hip.MoELayer(gate_up=gate_up, down=down, router=router, router_bias=bias, hidden=HIDDEN,
                                   inter=INTER, n_experts=EXPERTS, top_k=TOP_K, shared_gate_up=sgu,
                                   shared_down=sdn, shared_gate=sgate, shared_inter=INTER))
    return layers


class HipEvents:
    """hipEvent_t through ctypes on the HIP runtime torch itself loaded (so they live in torch's context)."""

    def __init__(self, torch):
        path = os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so")
        self.rt = ctypes.CDLL(path)
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        arr = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            assert self.rt.hipEventCreate(ctypes.byref(h)) == 0
            arr[i] = h
        return arr

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.rt.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, arr):
        for h in arr:
            self.rt.hipEventDestroy(h)


def stage_bytes(stage, T, U, shared=True):
    """Algorithmic HBM bytes of one stage for T tokens whose routing touches U distinct experts."""
    P = T * TOP_K
    S = 1 if shared else 0
    if stage == "router":
        return ROUTER_BYTES + HIDDEN * 4 + T * HIDDEN * 4 + T * EXPERTS * 4
    if stage == "gate_up":
        return (U + S) * GATE_UP_BYTES + T * HIDDEN * 4 + (P + T * S) * INTER * 4
    if stage == "down":
        return (U + S) * DOWN_BYTES + (P + T * S) * (INTER + HIDDEN) * 4
    if stage == "combine":
        return (P + T * S) * HIDDEN * 4 + T * HIDDEN * 4
    return 0


def layer_bytes(T, U):
    """The touched bytes of a layer for T tokens: the touched experts (U routed + the shared one), the fp32 router
    and shared gate, x and y."""
    return (U + 1) * EXPERT_BYTES + ROUTER_BYTES + HIDDEN * 4 + T * HIDDEN * 4 * 2


def unique_experts(torch, layers, xs, T):
    """Distinct experts per layer for each input set, from an eager run that returns the routing."""
    counts = []
    for xset in xs:
        for l, layer in enumerate(layers):
            ids = torch.empty(T, TOP_K, dtype=torch.int32, device="cuda")
            layer(xset[l], ids=ids)
            counts.append(ids)
    torch.cuda.synchronize()
    return [int(torch.unique(ids).numel()) for ids in counts]


def run_decode(torch, hip, layers, T, steps, warmup, n_sets, label, graph=True):
    """One step = T tokens through every layer; returns timings and byte counts. graph=False launches the layers
    eagerly (for counter collection, which sees dispatches made outside graphs). A split-plan step (batched
    decode) always runs eagerly, its layers inside one fork scope: the layers' MFMA experts run on the library's
    second stream and meet the caller's stream through the workspace, and a graph replay starts the second
    stream's kernels late (64 tokens, Zipf routing, 40 layers: 93 us per layer replayed against 85 launched)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1000 + T)
    L = len(layers)
    xs = [torch.randn(L, T, HIDDEN, device="cuda", generator=gen) for _ in range(n_sets)]
    ys = torch.empty(L, T, HIDDEN, device="cuda")
    ws = new_workspace(max(layer.workspace_bytes(T) for layer in layers), "cuda")
    # a split-plan step runs its layers in one fork scope: the MFMA experts' hand-offs to the second stream go
    # through the workspace, with one fork and one join for the whole step
    split = layers[0].plan(T) == "split"
    scope = hip.fork_scope if split else contextlib.nullcontext
    graph = graph and not split

    def all_layers(xset):
        with scope():
            for l, layer in enumerate(layers):
                layer(xset[l], out=ys[l], workspace=ws)

    graphs = []
    capture = torch.cuda.Stream()
    for xset in xs:
        all_layers(xset)  # warm the kernels once outside capture
        torch.cuda.synchronize()
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=capture):
                all_layers(xset)
            graphs.append(g)
    torch.cuda.synchronize()

    def step(i):
        if graph:
            graphs[i % n_sets].replay()
        else:
            all_layers(xs[i % n_sets])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end)
    assert torch.isfinite(ys).all(), f"{label}: non-finite outputs"
    checks = {}
    if split:
        # a fork-scope hand-off that gave up would skip the MFMA experts (stale outputs, little change in time):
        # the workspace's status must be clean, and the last timed step must equal per-call runs bit for bit
        st = layers[0].status(ws)
        if st != 0:
            raise SystemExit(f"{label}: a fork-scope wait gave up during the timed steps (status {st})")
        last = xs[(steps - 1) % n_sets]
        own = new_workspace(max(layer.workspace_bytes(T) for layer in layers), "cuda")
        ref = torch.stack([layer(last[l], workspace=own) for l, layer in enumerate(layers)])
        torch.cuda.synchronize()
        if not torch.equal(ref, ys):
            raise SystemExit(f"{label}: the timed step differs from per-call runs "
                             f"(max diff {(ref - ys).abs().max().item():.3e})")
        checks = {"status_after_timed_steps": st, "timed_step_equals_per_call_runs": True}
        del ref, own
    U = unique_experts(torch, layers, xs, T)
    us_layer = ms * 1000.0 / (steps * L)
    bytes_layer = sum(layer_bytes(T, u) for u in U) / len(U)
    log(f"{label}: {ms / steps:.3f} ms/step, {us_layer:.2f} us/layer, {us_layer / T:.3f} us/token/layer, "
        f"{bytes_layer / us_layer / 1e3:.0f} GB/s, mean unique experts {sum(U) / len(U):.1f}")
    del graphs
    return {"ms_per_step": ms / steps, "wall_s": wall, "us_per_layer": us_layer, "us_per_token_layer": us_layer / T,
            "bytes_per_layer": bytes_layer, "hbm_gbps": bytes_layer / us_layer / 1e3, "unique": U, "xs": xs,
            "ws": ws, "launch": "hipGraph replay" if graph else ("eager, one fork scope per step" if split else "eager"),
            **checks}


def profile_stages(torch, hip, layers, xs, T, ws, reps=2):
    """Per-stage durations of the layer from HIP events recorded between its kernels (eager, same stream)."""
    ev = HipEvents(torch)
    n_st = hip.library().wl_moe_stage_count()
    names = [hip.library().wl_moe_stage_name(i).decode() for i in range(n_st)]
    calls = []
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.empty(T, HIDDEN, device="cuda")
    for _ in range(reps):
        for xset in xs:
            for l, layer in enumerate(layers):
                events = ev.create(n_st + 1)
                x = xset[l].contiguous()
                hip.check(hip.library().wl_moe_layer_profile(ctypes.byref(layer.struct), x.data_ptr(), T,
                                                             out.data_ptr(), None, None, ws.data_ptr(), ws.numel(),
                                                             stream, events))
                calls.append(events)
    torch.cuda.synchronize()
    per = {n: [] for n in names}
    for events in calls:
        for i, n in enumerate(names):
            per[n].append(ev.elapsed_ms(events[i], events[i + 1]) * 1000.0)
        ev.destroy(events)
    return {n: sum(v) / len(v) for n, v in per.items()}


def rms_norm_torch(torch, x, w, eps=1e-6):
    """engines/base.py:27-31, zero-centered (x * rsqrt(mean(x^2) + eps) * (1 + w)), in torch fp32: the input of
    the next-layer guess (it only feeds a routing guess, so torch's own rounding is fine here)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w)


def run_chained(torch, hip, layers, steps, warmup, n_sets):
    """Decode b=1 with each layer's input the previous layer's output, as the model chains them:
    x_{l+1} = x_l + MoE_l(rms_norm_l(x_l)) (engines/qwen36/model.py:22; the attention half is not part of this
    path). One launch per layer (the layer's pre-norm and residual flags), the stack captured as one graph per
    starting vector and replayed; the graph's output is checked bit for bit against an eager pass. Timed twice in
    the same session: without and with the next-layer guess (WL_MOE_GUESS_NEXT: layer l also computes layer l+1's
    router on rms_norm_{l+1}(x_l), the reference's guess_next_layer, engines/base.py:392-406 with
    engines/qwen36/model.py:30-31, and pulls the guessed experts' gate_up rows into the caches); both give the same
    bits. Also measures how often that guess names layer l+1's actual experts."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4242)
    L = len(layers)
    norm_w = [torch.randn(HIDDEN, device="cuda", generator=gen) * 0.1 for _ in range(L)]
    chain = [layer.with_norm(norm_w[l]) for l, layer in enumerate(layers)]
    x0 = [torch.randn(1, HIDDEN, device="cuda", generator=gen) for _ in range(n_sets)]
    xs = torch.empty(L, 1, HIDDEN, device="cuda")  # layer l writes x_{l+1} into xs[l]
    ws = new_workspace(max(layer.workspace_bytes(1) for layer in chain), "cuda")

    def stack(x, ids=None):
        for l, layer in enumerate(chain):
            layer(x if l == 0 else xs[l - 1], out=xs[l], workspace=ws, ids=None if ids is None else ids[l])

    ids = torch.empty(n_sets, L, 1, TOP_K, dtype=torch.int32, device="cuda")

    def measure(guess):
        # the last layer's next is the first (the next step's layer 0, whose input is a new token: no guess there)
        for l in range(L):
            chain[l].set_next(chain[(l + 1) % L], guess=guess and l + 1 < L)
        eager_out = []
        for s in range(n_sets):
            stack(x0[s], ids[s])
            eager_out.append(xs[L - 1].clone())
        torch.cuda.synchronize()
        graphs = []
        capture = torch.cuda.Stream()
        for s in range(n_sets):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=capture):
                stack(x0[s])
            graphs.append(g)
        for s in range(n_sets):
            graphs[s].replay()
            torch.cuda.synchronize()
            assert torch.equal(xs[L - 1], eager_out[s]), "chained decode: graph replay differs from the eager pass"
        for i in range(warmup):
            graphs[i % n_sets].replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            graphs[i % n_sets].replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        assert torch.isfinite(xs).all(), "chained decode: non-finite outputs"
        status = chain[0].status(ws)
        assert status == 0, f"chained decode: workspace status {status} after the timed steps"
        del graphs
        return ms, eager_out

    ms_plain, out_plain = measure(False)
    ms_guess, out_guess = measure(True)
    for s in range(n_sets):
        assert torch.equal(out_plain[s], out_guess[s]), "chained decode: the next-layer guess changed the outputs"
    hits = []
    for s in range(n_sets):  # the routing of every layer (ids of the last eager pass of each set), then the guess
        stack(x0[s], ids[s])
        for l in range(L - 1):
            x_l = x0[s] if l == 0 else xs[l - 1]
            _, guess, _ = layers[l + 1].route(rms_norm_torch(torch, x_l, norm_w[l + 1]))
            hits.append(torch.isin(guess[0], ids[s, l + 1, 0]).sum())
    torch.cuda.synchronize()
    hits = torch.stack(hits)
    hit_rate = float(hits.sum()) / (len(hits) * TOP_K)
    all_hit = float((hits == TOP_K).float().mean())  # layers whose experts the guess names all of
    for layer in chain:
        layer.set_next(None)
    us_plain = ms_plain * 1000.0 / (steps * L)
    us_guess = ms_guess * 1000.0 / (steps * L)
    bytes_layer = layer_bytes(1, TOP_K)
    log(f"decode b=1 chained: {us_plain:.2f} us/layer ({bytes_layer / us_plain / 1e3:.0f} GB/s); with the next-layer "
        f"guess {us_guess:.2f} us/layer; guess hit rate {hit_rate:.3f}")
    return {"us_per_token_layer": round(us_plain, 3), "ms_per_step": round(ms_plain / steps, 4),
            "hbm_gbps": round(bytes_layer / us_plain / 1e3, 1), "steps": steps, "starting_vectors": n_sets,
            "graph_matches_eager": True, "next_layer_guess_hit_rate": round(hit_rate, 4),
            "next_layer_guess_all_hit": round(all_hit, 4),
            "guess": "top-8 of layer l+1's router on rms_norm_{l+1}(x_l), scored against layer l+1's experts",
            "with_next_layer_guess": {"us_per_token_layer": round(us_guess, 3), "same_outputs": True,
                                      "flag": "WL_MOE_GUESS_NEXT (guessed experts' gate_up rows pulled into L2)"},
            "norm": "zero-centered RMSNorm, weights N(0, 0.1), eps 1e-6"}


def routing_margins(torch, logits):
    """Per-token gap between the 8th and 9th largest router logits over the [N, E] logits of a workload, and the
    tokens whose 8th and 9th fp32 softmax probabilities are equal: the reference selects on probabilities
    (engines/base.py:93-94), where exp rounding can tie distinct logits that the logit-based selection orders."""
    top = torch.topk(logits, TOP_K + 1, dim=-1).values
    m = (top[:, TOP_K - 1] - top[:, TOP_K]).float()
    probs = torch.topk(torch.softmax(logits, dim=-1), TOP_K + 1, dim=-1).values
    return {"tokens": int(m.numel()), "min": float(m.min()), "p1": float(torch.quantile(m, 0.01)),
            "median": float(m.median()), "logit_ties": int((m == 0).sum()),
            "prob_ties": int((probs[:, TOP_K - 1] == probs[:, TOP_K]).sum())}


def layer_logits(torch, layers, inputs):
    """Router logits of layers[l] on inputs[l] for every l, concatenated."""
    out = [layer.route(x, return_logits=True)[3] for layer, x in zip(layers, inputs)]
    return torch.cat(out)


def run_small_configs(torch, hip, reps=5):
    """The single-matrix and single-expert workloads on the GPU, each call on its own copy of the weights so the
    256 MB MALL cannot serve repeats: 1024 copies of the 512 x 2048 Q4_K matrix (604 MB) through wl_gemv, and 256
    copies of one expert (gate/up Q4_K 512 x 2048, down Q6_K 2048 x 512; 522 MB) through wl_moe_layer as a
    one-expert, top-1 layer without a shared expert (its router is a 2048-value dot product and its routing
    weight 1). All calls of a workload are captured in one graph, replayed `reps` times; figures are per call."""
    lib = hip.library()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)

    def timed(fn, calls):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1000.0 / (reps * calls)

    n0, rows, k = 1024, 512, 2048
    w0 = gen_q4k(torch, n0 * rows * (k // 256), gen).view(n0, -1)
    x0 = torch.randn(1, k, device="cuda", generator=gen)
    y0 = torch.empty(n0, rows, device="cuda")

    def gemvs():
        stream = torch.cuda.current_stream().cuda_stream
        for i in range(n0):
            hip.check(lib.wl_gemv(12, w0[i].data_ptr(), rows, k, Q4K_ROW, x0.data_ptr(), 1, y0[i].data_ptr(),
                                  stream))

    us0 = timed(gemvs, n0)
    c0_bytes = 600064
    del w0
    n1 = 256
    gate_up = gen_q4k(torch, n1 * 2 * INTER * (HIDDEN // 256), gen).view(n1, -1)
    down = gen_q6k(torch, n1 * HIDDEN * (INTER // 256), gen).view(n1, -1)
    router = torch.randn(1, HIDDEN, device="cuda", generator=gen) * 0.02
    experts = [hip.MoELayer(gate_up=gate_up[i:i + 1], down=down[i:i + 1], router=router, hidden=HIDDEN,
                            inter=INTER, n_experts=1, top_k=1) for i in range(n1)]
    x1 = torch.randn(1, HIDDEN, device="cuda", generator=gen)
    y1 = torch.empty(n1, 1, HIDDEN, device="cuda")
    ws = new_workspace(experts[0].workspace_bytes(1), "cuda")

    def expert_calls():
        for i, e in enumerate(experts):
            e(x1, out=y1[i], workspace=ws)

    us1 = timed(expert_calls, n1)
    c1_bytes = 2056192
    assert torch.isfinite(y0).all() and torch.isfinite(y1).all()
    log(f"config 0 (Q4_K GEMV 512x2048): {us0:.2f} us/call, {c0_bytes / us0 / 1e3:.0f} GB/s; config 1 (one "
        f"expert, b=1, {experts[0].plan(1)}): {us1:.2f} us/call, {c1_bytes / us1 / 1e3:.0f} GB/s")
    return {"config0_gemv": {"us_per_call": round(us0, 3), "bytes": c0_bytes, "gbps": round(c0_bytes / us0 / 1e3, 1),
                             "weight_copies": n0, "rotated_mb": round(n0 * rows * Q4K_ROW / 1e6, 1)},
            "config1_expert": {"us_per_call": round(us1, 3), "bytes": c1_bytes,
                               "gbps": round(c1_bytes / us1 / 1e3, 1), "weight_copies": n1,
                               "rotated_mb": round(n1 * EXPERT_BYTES / 1e6, 1), "plan": experts[0].plan(1)},
            "graph": f"all calls of a workload in one graph, {reps} replays"}


def measured_traffic(kernel):
    """HBM bytes per dispatch of `kernel` from the committed counter summary (rocprofv3 FETCH_SIZE and WRITE_SIZE
    runs of this script, each scaled by the same counter's reading for a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_decode_b1_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_dispatch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_info():
    """The host's CPU model (lscpu, else /proc/cpuinfo) and counts."""
    import subprocess
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None and os.path.exists("/proc/cpuinfo"):
        model = next((l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")), None)
    return {"model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_baseline():
    """The CPU oracle (numpy dequantize of the touched weights, then fp32 BLAS matmuls, fp32 router and combine;
    the reference's CPU path gguf/quants.py + matmul restated) on this host, for each workload:
      config 0: the 512 x 2048 Q4_K GEMV (seed 0), repeated for >= 0.5 s;
      config 1: one expert at batch 1 (seed 0), repeated for >= 0.5 s;
      config 2: the full layer (seed 1) at batch 1, >= 8 tokens over >= 3 s, each a new token;
      config 3: 64 tokens through 40 layer passes with Zipf(1.1) routing; the passes share the seed-1 expert
                weights (the oracle dequantizes from the quantized bytes on every pass, so sharing saves no work)
                and each draws its own Zipf permutation and tokens;
      config 4: one layer x 4096 tokens, timed once, extrapolated x40 to the 40-layer chunk.
    Threads: the BLAS pool and torch use the host's CPU share (OMP_NUM_THREADS when set, as on machines that
    allot a share of their cores to each GPU, else os.cpu_count())."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info, threadpool_limits

    from gguf import synth
    from oracle import moe_ref
    from oracle.quants_ref import dequantize_matrix
    n_threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count())
    torch.set_num_threads(n_threads)
    out = {}
    with threadpool_limits(limits=n_threads, user_api="blas"):
        blas = max([p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"] or [1])

        def repeat(fn, min_s, min_n=3):  # one untimed call first (page faults, pool start-up)
            fn(-1)
            n, t0 = 0, time.perf_counter()
            while n < min_n or time.perf_counter() - t0 < min_s:
                fn(n)
                n += 1
            return (time.perf_counter() - t0) / n, n

        c0 = synth.gemv_case(0)
        dt, n = repeat(lambda i: c0["x"] @ dequantize_matrix(c0["w"], "Q4_K", 512, 2048).T, 0.5)
        out["config0_gemv"] = {"us_per_call": round(dt * 1e6, 1), "calls": n, "gbps": round(600064 / dt / 1e9, 3)}
        c1 = synth.expert_case(0)

        def expert(i):
            gu = np.concatenate((dequantize_matrix(c1["gate"], "Q4_K", 512, 2048),
                                 dequantize_matrix(c1["up"], "Q4_K", 512, 2048)))
            moe_ref.expert_ffn(c1["x"], gu, dequantize_matrix(c1["down"], "Q6_K", 2048, 512), 512)
        dt, n = repeat(expert, 0.5)
        out["config1_expert"] = {"us_per_call": round(dt * 1e6, 1), "calls": n,
                                 "gbps": round(2056192 / dt / 1e9, 3)}
        lw = synth.moe_layer(1)
        dt, n = repeat(lambda i: moe_ref.layer(synth.tokens(11 + i, 1), lw), 3.0, 8)
        out["config2_decode_b1"] = {"us_per_token_layer": round(dt * 1e6, 1), "tokens": n,
                                    "gbps": round(layer_bytes(1, TOP_K) / dt / 1e9, 3)}
        rng = np.random.default_rng(3)
        t3, unique = 0.0, []
        for p in range(LAYERS):
            lz = dict(lw, router_bias=synth.zipf_bias(rng, EXPERTS, 1.1))
            x = synth.tokens(100 + p, 64)
            t0 = time.perf_counter()
            _, ids, _, _ = moe_ref.layer(x, lz, return_routing=True)
            t3 += time.perf_counter() - t0
            unique.append(len(np.unique(ids)))
        out["config3_decode_b64"] = {"us_per_token_layer": round(t3 / (LAYERS * 64) * 1e6, 1),
                                     "ms_per_step": round(t3 * 1e3, 1), "layers": LAYERS,
                                     "mean_unique_experts": round(float(np.mean(unique)), 1)}
        x = synth.tokens(7, 4096)
        t0 = time.perf_counter()
        moe_ref.layer(x, lw)
        t4 = time.perf_counter() - t0
        out["config4_prefill_4096"] = {"ms_per_layer": round(t4 * 1e3, 1),
                                       "ms_per_chunk_extrapolated_x40": round(t4 * 1e3 * LAYERS, 1),
                                       "tok_per_s": round(4096 / (t4 * LAYERS), 2), "timed_layers": 1}
    us = out["config2_decode_b1"]["us_per_token_layer"]
    return {"value": us, "unit": "us/token/layer", "cores": n_threads, "kind": "port",
            "sample": f"config 2 line: {out['config2_decode_b1']['tokens']} decode tokens (b=1) through one "
                      "full-shape layer (256 experts, top-8, shared; seed-1 weights), numpy dequantize + fp32 BLAS "
                      "matmul; per-config figures in configs",
            "hbm_equiv_gbps": round(layer_bytes(1, TOP_K) / us / 1e3, 3),
            "threads": {"torch_get_num_threads": torch.get_num_threads(), "blas_threads": int(blas),
                        "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")},
            "cpu": cpu_info(), "configs": out}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--sets", type=int, default=8, help="distinct input sets (graphs) cycled through")
    ap.add_argument("--skip-b64", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-load", action="store_true")
    ap.add_argument("--skip-linear", action="store_true")
    ap.add_argument("--skip-chained", action="store_true")
    ap.add_argument("--skip-small", action="store_true", help="skip the GPU timings of configs 0 and 1")
    ap.add_argument("--load-layers", type=int, default=8,
                    help="full-shape layers in the synthetic GGUF file of the loader measurement")
    ap.add_argument("--no-next", action="store_true",
                    help="decode without the next-layer overlap (WlMoeLayer.next unset)")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the decode layers eagerly instead of replaying HIP graphs (for counter runs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB five times (the reference kernel for "
                         "scaling FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the MoE layer here runs on a single MI355X (expert-parallel "
              "sharding across GPUs is designed, not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 5}), flush=True)
        return
    from gguf import hip
    hip.library()

    log(f"building {args.layers} layers in HBM")
    t = time.time()
    layers = build_layers(torch, hip, args.layers)
    if not args.no_next:  # each layer names the one run after it (the step loops back to layer 0)
        for i, layer in enumerate(layers):
            layer.set_next(layers[(i + 1) % len(layers)])
    torch.cuda.synchronize()
    log(f"built in {time.time() - t:.1f}s, {torch.cuda.memory_allocated() / 1e9:.1f} GB allocated")

    d1 = run_decode(torch, hip, layers, 1, args.steps, args.warmup, args.sets, "decode b=1",
                    graph=not args.no_graph)
    stages = profile_stages(torch, hip, layers, d1["xs"], 1, d1["ws"])
    U1 = sum(d1["unique"]) / len(d1["unique"])
    plan = layers[0].plan(1)
    if plan == "fused":  # one launch holds every stage: the events around it (eager) include the launch latency
        log(f"b=1 fused kernel, events around single eager launches: {stages['router']:.2f} us per layer")
    else:
        log("stage us (b=1): " + ", ".join(f"{k} {v:.2f}" for k, v in stages.items()))
    if plan == "fused":
        # one kernel holds the whole layer, so the timed region is that kernel back to back: its events (on the
        # stream the graphs replay on) over the launch count give the launch duration, gaps between launches
        # included. The events around single eager launches also hold the launch latency.
        dominant, dom_bytes, dom_us = "k_moe_decode", layer_bytes(1, U1), d1["us_per_layer"]
        stages = {"k_moe_decode": dom_us, "k_moe_decode_eager_events": stages["router"]}
    else:  # the stage moving the most bytes
        dominant = max(("router", "gate_up", "down", "combine"), key=lambda n: stage_bytes(n, 1, U1))
        dom_bytes, dom_us = stage_bytes(dominant, 1, U1), stages[dominant]
    achieved = dom_bytes / dom_us / 1e3  # GB/s
    result = {
        "metric": METRIC,
        "value": round(d1["us_per_token_layer"], 3),
        "unit": "us/token/layer",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(d1["ms_per_step"], 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"decode b=1 through {args.layers} stacked Qwen3.6-35B-A3B MoE layers (hidden 2048, "
                               "256 experts x width 512, top-8, shared expert; gate/up Q4_K, down Q6_K, fp32 "
                               "router), all experts HBM-resident",
                   "layers": args.layers, "tokens_per_step": 1, "input_sets": args.sets, "graph": "hipGraph"},
        "hbm_gbps": round(d1["hbm_gbps"], 1),
        "hbm_frac": round(d1["hbm_gbps"] / HBM_PEAK_GBPS, 4),
        "stages_us_b1": {k: round(v, 3) for k, v in stages.items()},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(dominant), "algorithmic_bytes": int(dom_bytes)},
    }
    margins = {"config2_decode_b1": routing_margins(
        torch, torch.cat([layer_logits(torch, layers, xset) for xset in d1["xs"]]))}
    del d1
    if not args.skip_chained:
        result["decode_b1_chained"] = run_chained(torch, hip, layers, args.steps, args.warmup, args.sets)
    if not args.skip_prefill:
        result["prefill"], x_prefill = run_prefill(torch, hip, layers, 4096, steps=2)
        margins["config4_prefill_4096"] = routing_margins(torch, layer_logits(torch, layers, [x_prefill] * len(layers)))
        del x_prefill
    if not args.skip_b64:
        del layers
        torch.cuda.empty_cache()
        zl = build_layers(torch, hip, args.layers, zipf=True, seed=3)
        d64 = run_decode(torch, hip, zl, 64, max(10, args.steps // 10), max(2, args.warmup // 4), 4, "decode b=64",
                         graph=not args.no_graph)
        result["decode_b64"] = {"us_per_token_layer": round(d64["us_per_token_layer"], 3),
                                "us_per_layer": round(d64["us_per_layer"], 2),
                                "hbm_gbps": round(d64["hbm_gbps"], 1),
                                "mean_unique_experts": round(sum(d64["unique"]) / len(d64["unique"]), 1),
                                "routing": "Zipf(1.1) router bias", "plan": zl[0].plan(64), "launch": d64["launch"],
                                "status_after_timed_steps": d64.get("status_after_timed_steps"),
                                "timed_step_equals_per_call_runs": d64.get("timed_step_equals_per_call_runs")}
        margins["config3_decode_b64"] = routing_margins(
            torch, torch.cat([layer_logits(torch, zl, xset) for xset in d64["xs"]]))
        del d64, zl
        torch.cuda.empty_cache()
    result["routing_margins"] = margins
    if not args.skip_small:
        result["small_configs_gpu"] = run_small_configs(torch, hip)
    if not args.skip_load:
        result["gguf_load"] = run_gguf_load(torch, args.load_layers)
    if not args.skip_linear:
        result["linear_q4k"] = run_linear(torch, hip)
    if not args.skip_cpu:
        log("timing the CPU oracle")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


def run_prefill(torch, hip, layers, T, steps):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    x = torch.randn(T, HIDDEN, device="cuda", generator=gen)
    ws = new_workspace(max(layer.workspace_bytes(T) for layer in layers), "cuda")
    y = torch.empty(T, HIDDEN, device="cuda")
    layers[0](x, out=y, workspace=ws)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        for layer in layers:
            layer(x, out=y, workspace=ws)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = len(layers) * T * (TOP_K + 1) * 3 * 2 * HIDDEN * INTER
    log(f"prefill T={T}: {ms:.1f} ms per chunk of {len(layers)} layers, {T / ms * 1e3:.0f} tok/s")
    return {"tokens": T, "ms_per_chunk": round(ms, 2), "tok_per_s": round(T / ms * 1e3, 1),
            "tflops": round(flops / ms / 1e9, 2), "mfma_frac": round(flops / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
            "path": layers[0].plan(T) + ": tiled fp32 router, bf16 MFMA grouped expert GEMMs (in-register "
                    "Q4_K/Q6_K dequant), fp32 combine"}, x


def run_linear(torch, hip, rows=2048, k=2048, T=4096, reps=20):
    """A quantized non-expert weight in a 4096-token prefill: GGMLWeight's F.linear above 8 tokens (its bf16 values
    dequantized once and kept, then the library's bf16 GEMM), wl_linear (bf16 MFMA with the weights dequantized in
    registers, nothing kept) and the reference's form (dequantize_gpu to bf16 on every call, then a bf16 matmul;
    gguf/metal.py:407), each as `reps` calls in one graph replay."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    raw = gen_q4k(torch, rows * (k // 256), gen).view(-1)
    x = torch.randn(T, k, device="cuda", generator=gen).to(torch.bfloat16)

    def timed(fn):
        # `reps` calls captured in one graph and replayed, so the figure is GPU time, not Python dispatch (the
        # first call, outside the capture, also builds GGMLWeight's kept bf16 values)
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1000.0 / reps

    weight = hip.GGMLWeight(raw, "Q4_K", (rows, k))
    us_kept = timed(lambda: torch.nn.functional.linear(x, weight))
    us_mfma = timed(lambda: hip.linear_mfma(raw, "Q4_K", (rows, k), x))
    us_ref = timed(lambda: torch.nn.functional.linear(x, hip.dequantize_gpu(raw, "Q4_K", (rows, k))))
    # the vendor library's bf16 GEMM alone on the same shape (the weight dequantized beforehand, outside the timing):
    # what this problem size allows a tuned dense GEMM
    wb = hip.dequantize_gpu(raw, "Q4_K", (rows, k))
    us_gemm = timed(lambda: torch.nn.functional.linear(x, wb))
    flops = 2.0 * T * rows * k
    log(f"linear Q4_K {rows}x{k}, {T} tokens: GGMLWeight F.linear (bf16 kept) {us_kept:.1f} us "
        f"({flops / us_kept / 1e6:.0f} TFLOP/s), wl_linear {us_mfma:.1f} us ({flops / us_mfma / 1e6:.0f} TFLOP/s), "
        f"dequantize + bf16 matmul per call {us_ref:.1f} us, the bf16 matmul alone {us_gemm:.1f} us "
        f"({flops / us_gemm / 1e6:.0f} TFLOP/s)")
    return {"rows": rows, "k": k, "tokens": T, "us_ggml_linear_kept": round(us_kept, 2),
            "tflops_ggml_linear_kept": round(flops / us_kept / 1e6, 1), "us_wl_linear": round(us_mfma, 2),
            "us_dequantize_matmul": round(us_ref, 2), "tflops_wl_linear": round(flops / us_mfma / 1e6, 1),
            "us_bf16_matmul_alone": round(us_gemm, 2), "tflops_bf16_matmul_alone": round(flops / us_gemm / 1e6, 1)}


def run_gguf_load(torch, n_layers):
    """GGUF file -> HBM: a synthetic Qwen3.6-shaped GGUF of n_layers MoE layers (random block bytes; the loader
    does not look at them) is written to a temporary directory and loaded with gguf.loader.load_experts. The file
    was just written, so it is read from the page cache: the figure is the loader's host-to-HBM rate, compared with
    a plain pinned host-to-device copy of 256 MiB timed the same way."""
    import shutil
    import tempfile

    import numpy as np
    from gguf import loader
    from gguf.writer import write_gguf

    rng = np.random.default_rng(9)
    arch = "qwen35moe"
    meta = {"general.architecture": arch, f"{arch}.block_count": n_layers, f"{arch}.embedding_length": HIDDEN,
            f"{arch}.expert_count": EXPERTS, f"{arch}.expert_used_count": TOP_K}
    # one layer's random bytes, written for every layer (the content does not matter to the loader)
    gate = rng.integers(0, 256, (EXPERTS, GATE_UP_BYTES // 2), dtype=np.uint8)
    up = rng.integers(0, 256, (EXPERTS, GATE_UP_BYTES // 2), dtype=np.uint8)
    down = rng.integers(0, 256, (EXPERTS, DOWN_BYTES), dtype=np.uint8)
    tensors = []
    for n in range(n_layers):
        tensors += [(f"blk.{n}.ffn_gate_exps.weight", "Q4_K", (EXPERTS, INTER, HIDDEN), gate),
                    (f"blk.{n}.ffn_up_exps.weight", "Q4_K", (EXPERTS, INTER, HIDDEN), up),
                    (f"blk.{n}.ffn_down_exps.weight", "Q6_K", (EXPERTS, HIDDEN, INTER), down)]
    folder = tempfile.mkdtemp(prefix="wl_gguf_")
    try:
        path = os.path.join(folder, "synthetic-moe.gguf")
        write_gguf(path, meta, tensors)
        del tensors
        header = loader.read_gguf(path)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        store = loader.load_experts(header, "cuda")
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        # spot check: first, middle and last expert of every layer, byte for byte
        for l in store.layers:
            for e in (0, EXPERTS // 2, EXPERTS - 1):
                gu = l.gate_up[e].cpu().numpy()
                half = GATE_UP_BYTES // 2
                assert np.array_equal(gu[:half], gate[e]) and np.array_equal(gu[half:], up[e])
                assert np.array_equal(l.down[e].cpu().numpy(), down[e])
        nbytes = store.loaded_bytes
        del store
    finally:
        shutil.rmtree(folder, ignore_errors=True)
    host = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    dev = torch.empty_like(host, device="cuda")
    dev.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(4):
        dev.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    copy_gbps = 4 * host.numel() / (time.perf_counter() - t0) / 1e9
    gbps = nbytes / dt / 1e9
    log(f"GGUF -> HBM: {nbytes / 1e9:.2f} GB of experts ({n_layers} layers) in {dt:.2f} s, {gbps:.1f} GB/s "
        f"(pinned copy {copy_gbps:.1f} GB/s)")
    return {"layers": n_layers, "bytes": nbytes, "seconds": round(dt, 3), "gbps": round(gbps, 2),
            "pinned_copy_gbps": round(copy_gbps, 2), "frac_of_pinned_copy": round(gbps / copy_gbps, 3),
            "source": "page cache (file just written)"}


if __name__ == "__main__":
    main()
