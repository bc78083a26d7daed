"""Benchmark: Mixtral-8x7B-shape MoE layer forward on one MI355X.

Workload (one step = one layer forward over one batch, inputs resident in HBM):
hidden 4096, 8 experts, top-2 softmax routing (renormalised), SwiGLU ffn
14336, bf16, router 4096x8 with a fixed per-expert fp32 logit bias N(0, 0.5^2)
for mildly skewed load; activations N(0,1), weights N(0, 0.02), synthetic.
The headline runs at 4096 tokens; decode sizes 1, 16 and 256 tokens are
reported alongside.

Prints one JSON line (rank 0): tokens/s for the whole layer, the roofline of
the dominant kernel (the grouped gate|up GEMM, MFMA bound) from HIP events on
the stream the kernels run on, per-stage times, HBM fractions of the decode
sizes, and the CPU baseline: the reference's torch-CPU forward restated in
oracle/ref_torch.py, timed on this host on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer tokens/s + grouped-GEMM % MFMA peak, Mixtral-8x7B shape bf16"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
H, E, K, I = 4096, 8, 2, 14336


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--decode", type=str, default="1,16,256",
                    help="comma-separated token counts reported beside the headline ('' = none)")
    ap.add_argument("--configs", type=str, default="phi35moe,finegrained,offload,norm_router",
                    help="other workloads reported beside the headline ('' = none)")
    ap.add_argument("--offload-layers", type=int, default=32)
    ap.add_argument("--offload-steps", type=int, default=256)
    ap.add_argument("--offload-tokens", type=int, default=8)
    ap.add_argument("--offload-host-pools", type=int, default=4,
                    help="distinct layers' experts staged in pinned memory (at most 4); deeper "
                         "layers reuse them")
    ap.add_argument("--offload-modes", type=str, default="",
                    help="comma-separated offload forward/residency modes (default: all of "
                         "bench.OFFLOAD_MODES)")
    ap.add_argument("--cpu-sample-tokens", type=int, default=4096)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--profile", type=int, default=0,
                    help="profiling aid: run only the layer at this many tokens")
    ap.add_argument("--profile-shape", type=str, default="mixtral",
                    choices=("mixtral", "phi35moe", "finegrained"),
                    help="profiling aid: the layer --profile runs (fine-grained: through "
                         "FusedMoE.forward with its 2 shared experts)")
    ap.add_argument("--copy-calib", type=int, default=0,
                    help="profiling aid: device-to-device copies of this many bytes, the "
                         "known-size reference for HBM byte counters")
    return ap.parse_args()


class Layer:
    """One MoE layer's weights (bf16, N(0, 0.02), generated on the GPU) and
    the libmoe355 stage calls of its forward. Default: the Mixtral shape with
    a fixed per-expert router bias N(0, 0.5^2)."""

    def __init__(self, dev, seed=0, hidden=H, experts=E, top_k=K, ffn=I, bias=None):
        import torch

        from reframework_amd import synth

        self.H, self.E, self.K, self.I = hidden, experts, top_k, ffn
        g = torch.Generator(device=dev).manual_seed(seed)
        self.dev = dev
        self.gate = (torch.randn(experts, hidden, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        self.w1 = [(torch.randn(2 * ffn, hidden, generator=g, device=dev) * 0.02).to(torch.bfloat16)
                   for _ in range(experts)]
        self.w2 = [(torch.randn(hidden, ffn, generator=g, device=dev) * 0.02).to(torch.bfloat16)
                   for _ in range(experts)]
        self.bias = (synth.mixtral_router_bias(experts, seed) if bias is None else bias).to(dev)
        self.w1p = [w.data_ptr() for w in self.w1]
        self.w2p = [w.data_ptr() for w in self.w2]

    def inputs(self, T, seed=1):
        import torch

        g = torch.Generator(device=self.dev).manual_seed(seed)
        return torch.randn(T, self.H, generator=g, device=self.dev).to(torch.bfloat16)


STAGES = ("router", "permute", "gate_up", "down", "combine")


def run_layer(layer, x, bufs, events=None):
    """router, then the routed experts on the current stream. Without events
    the experts run as the layer runs them, one moe355_fused_experts call
    (permute -> gate_up -> down -> combine; at decode sizes the grouping
    happens inside gate_up). With events (the stage-timing pass: six events
    on the stream the kernels run on) the stages are called one by one with
    an event before the first and after each."""
    from reframework_amd import _capi

    plan, ws, w, ids, out = bufs
    s = _capi.stream_handle(x.device)
    if events:
        events[0].record()
    _capi.router_topk(x, layer.gate, layer.bias, layer.K, True, True, 0, w, ids, stream=s)
    if not events:
        _capi.fused_experts(x, layer.w1p, layer.w2p, layer.I, w, ids, 0, out, ws, stream=s)
        return
    events[1].record()
    _capi.permute(plan, ids, ws, stream=s)
    events[2].record()
    _capi.gate_up(plan, x, layer.w1p, 0, ws, stream=s)
    events[3].record()
    _capi.down(plan, layer.w2p, ws, stream=s)
    events[4].record()
    _capi.combine(plan, w, out, False, ws, stream=s)
    events[5].record()


def make_bufs(layer, T):
    import torch

    from reframework_amd import _capi

    plan = _capi.make_plan(T, layer.H, layer.I, layer.E, layer.K, _capi.BF16)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=layer.dev)
    w = torch.empty(T, layer.K, dtype=torch.float32, device=layer.dev)
    ids = torch.empty(T, layer.K, dtype=torch.int32, device=layer.dev)
    out = torch.empty(T, layer.H, dtype=torch.bfloat16, device=layer.dev)
    return plan, ws, w, ids, out


def measure(layer, T, steps, warmup):
    """Whole-layer ms/step plus per-stage averages from HIP events."""
    import torch

    x = layer.inputs(T)
    bufs = make_bufs(layer, T)
    for _ in range(warmup):
        run_layer(layer, x, bufs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run_layer(layer, x, bufs)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    # stage timing pass (events between the stages, on the kernels' stream)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(steps)]
    for i in range(steps):
        run_layer(layer, x, bufs, events=ev[i])
    torch.cuda.synchronize()
    stage_ms = {name: sum(e[j].elapsed_time(e[j + 1]) for e in ev) / steps
                for j, name in enumerate(STAGES)}
    stage_ms.update(small_stage_ms(layer, x, bufs))
    ids = bufs[3].cpu().numpy()
    routed = sorted(set(int(v) for v in ids.reshape(-1)))
    plan, ws = bufs[0], bufs[1]
    tiles = int(ws[plan.off_tile_map:plan.off_tile_map + 4].cpu().view(torch.int32)[0])
    return {"ms": ms, "gate_up_ms": stage_ms["gate_up"], "down_ms": stage_ms["down"],
            "stage_ms": stage_ms, "layer_ev_ms": sum(stage_ms.values()),
            "routed_experts": len(routed), "plan_path": plan.path,
            "down_splits": plan.down_splits, "token_tiles": tiles}


def small_stage_ms(layer, x, bufs, reps=20):
    """ms per launch of the short stages (router, permute, combine): `reps`
    back-to-back launches of one stage between two events on the kernels'
    stream, queued behind three layer steps so the GPU never waits for the
    host. Each launch rewrites its outputs from unchanged inputs. Recording an
    event beside every launch of a 5-20 us kernel adds a few us of queue
    overhead per launch that the kernel itself does not spend."""
    import torch

    from reframework_amd import _capi

    plan, ws, w, ids, out = bufs
    s = _capi.stream_handle(x.device)
    fns = {
        "router": lambda: _capi.router_topk(x, layer.gate, layer.bias, layer.K, True, True, 0,
                                            w, ids, stream=s),
        "permute": lambda: _capi.permute(plan, ids, ws, stream=s),
        "combine": lambda: _capi.combine(plan, w, out, False, ws, stream=s),
    }
    res = {}
    for name, fn in fns.items():
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(3):
            run_layer(layer, x, bufs)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        b.synchronize()
        res[name] = a.elapsed_time(b) / reps
    return res


def rotating_pairs(layer, steps, warmup, rotate=True):
    """One token per step whose two experts change every step, cycling
    through the disjoint pairs (0,1), (2,3), (4,5), (6,7): an expert's weights
    come back every four steps, after 2.1 GB of other weights, so nothing of
    them survives in the 256 MB Infinity Cache (the plain decode bench
    repeats one routing each step). Times the routed-expert call alone (the
    router's output is replaced by these ids). rotate=False keeps the first
    pair every step, for comparison."""
    import torch

    from reframework_amd import _capi

    x = layer.inputs(1)
    pairs = [torch.tensor([[2 * p, 2 * p + 1]], dtype=torch.int32, device=layer.dev)
             for p in range(layer.E // 2)]
    w = torch.tensor([[0.6, 0.4]], dtype=torch.float32, device=layer.dev)
    out = torch.empty(1, layer.H, dtype=torch.bfloat16, device=layer.dev)
    plan = _capi.make_plan(1, layer.H, layer.I, layer.E, 2, _capi.BF16)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=layer.dev)

    def step(i):
        _capi.fused_experts(x, layer.w1p, layer.w2p, layer.I, w,
                            pairs[i % len(pairs) if rotate else 0], 0, out, ws)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    alg = 2 * 3 * layer.H * layer.I * 2 + 2 * layer.H * 2
    return {"ms": round(ms, 4), "alg_bytes": alg,
            "hbm_gb_s": round(alg / (ms / 1000.0) / 1e9, 1),
            "hbm_frac": round(alg / (ms / 1000.0) / 1e9 / PEAK_HBM_GBS, 4)}


def stage_rates(layer, T, m):
    """Algorithmic bytes and achieved GB/s of the HBM-bound stages (times per
    launch from small_stage_ms): the
    router (x and the gate read, T*K weights and ids written), the permute
    (it moves indices only: T*K ids read, slot_to_row / row_src and the
    per-block counts written; token rows are gathered by gate_up), and the
    combine (each routed slot's y row in the format the plan's down
    projection writes, the routing weights and slot map, the output)."""
    from reframework_amd import _capi

    plan = _capi.make_plan(T, layer.H, layer.I, layer.E, layer.K, _capi.BF16)
    R, H, E, K = T * layer.K, layer.H, layer.E, layer.K
    y_narrow = plan.path in (_capi.PATH_MFMA_TILED, _capi.PATH_MFMA_TILED128) and \
        plan.down_splits == 1
    y_bytes = R * H * 2 if y_narrow else plan.down_splits * R * H * 4
    alg = {"router": T * H * 2 + E * H * 2 + T * K * 8,
           "permute": R * 4 + 3 * R * 4 + plan.n_blocks * E * 4 + (E + 1) * 4,
           "combine": y_bytes + R * 8 + T * H * 2}
    out = {}
    for name, nbytes in alg.items():
        ms = m["stage_ms"][name]
        out[name] = {"us": round(ms * 1000.0, 2), "alg_bytes": nbytes,
                     "gb_s": round(nbytes / (ms / 1000.0) / 1e9, 1),
                     "hbm_frac": round(nbytes / (ms / 1000.0) / 1e9 / PEAK_HBM_GBS, 4)}
    out["gate_up"] = {"us": round(m["stage_ms"]["gate_up"] * 1000.0, 2)}
    out["down"] = {"us": round(m["stage_ms"]["down"] * 1000.0, 2)}
    return out


def usable_cores():
    """Cores this process may run on: its CPU affinity, capped by a cgroup
    CPU quota when one is set (a container's share of a larger host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "host CPU"


def cpu_baseline(layer, T):
    """The reference's resident forward restated in torch on the host CPU
    (oracle/ref_torch.py), on every core this process may use, in two
    variants: (i) faithful, stacking all experts into fresh banks on every
    call as the reference does, (ii) with the banks stacked once beforehand.
    Median of 3 runs after a warm-up, within a 30 s budget per variant;
    tokens/s = T / median. ``value`` is the faithful variant."""
    import torch

    from oracle import ref_torch

    cores = usable_cores()
    torch.set_num_threads(cores)
    gate = layer.gate.cpu()
    w1 = [w.cpu() for w in layer.w1]
    w2 = [w.cpu() for w in layer.w2]
    bias = layer.bias.cpu()
    x = layer.inputs(T).cpu()
    variants = {}
    with torch.no_grad():
        stacked = (torch.stack(w1), torch.stack(w2))
        for name, banks in (("faithful", None), ("pre_stacked", stacked)):
            ref_torch.forward(x[:8], gate, w1, w2, K, bias=bias, stacked=banks)  # warm-up
            times = []
            t_start = time.perf_counter()
            while len(times) < 3 and (time.perf_counter() - t_start) < 30.0:
                t0 = time.perf_counter()
                ref_torch.forward(x, gate, w1, w2, K, bias=bias, stacked=banks)
                times.append(time.perf_counter() - t0)
            times.sort()
            med = times[len(times) // 2]
            variants[name] = {"tokens_per_s": round(T / med, 1), "median_s": round(med, 4),
                              "runs": len(times)}
        del stacked
    model = cpu_model()
    return {"value": variants["faithful"]["tokens_per_s"], "unit": "tokens/s", "cores": cores,
            "kind": "port", "host_cpus": os.cpu_count(), "cpu_model": model,
            "variants": variants,
            "sample": f"reference resident forward restated in torch (oracle/ref_torch.py): "
                      f"Mixtral shape bf16, {T} tokens, {cores} threads on {model}; value = "
                      f"faithful variant (all experts stacked per call, median "
                      f"{variants['faithful']['median_s']:.2f} s); pre-stacked banks: "
                      f"{variants['pre_stacked']['tokens_per_s']:.0f} tokens/s"}


def measured_traffic(T):
    """HBM-side bytes per gate_up launch at this workload from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE profile (copy-calibrated), or None when
    no profile covers it. Counters cannot be read from inside the timed run."""
    path = os.path.join(ROOT, "profiles", "traffic_gate_up_mixtral_t4096.json")
    if T != 4096 or not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    return rec.get("traffic_bytes_per_launch")


def _rates(flops, alg_bytes, ms):
    sec = ms / 1000.0
    return {"tflops": round(flops / sec / 1e12, 2),
            "mfma_frac": round(flops / sec / 1e12 / PEAK_BF16_TFLOPS, 4),
            "hbm_gb_s": round(alg_bytes / sec / 1e9, 1),
            "hbm_frac": round(alg_bytes / sec / 1e9 / PEAK_HBM_GBS, 4)}


def config_phi35moe(dev, steps, warmup, T=2048):
    """Phi-3.5-MoE shape: hidden 4096, 16 experts, top-2, ffn 6400, 2048
    tokens, router bias log Zipf(1.1) over a seeded expert ranking."""
    import torch

    from reframework_amd import synth

    h, e, k, i = 4096, 16, 2, 6400
    layer = Layer(dev, hidden=h, experts=e, top_k=k, ffn=i, bias=synth.zipf_router_bias(e, 1.1))
    m = measure(layer, T, steps, warmup)
    flops = 6.0 * T * k * h * i + 2.0 * T * h * e
    alg = m["routed_experts"] * 3 * h * i * 2 + e * h * 2 + 2 * T * h * 2
    res = {"workload": "phi-3.5-moe-shape layer forward", "tokens": T, "hidden": h, "experts": e,
           "top_k": k, "ffn": i, "ms": round(m["ms"], 4),
           "tokens_per_s": round(T / (m["ms"] / 1000.0), 1), "routed_experts": m["routed_experts"],
           "gate_up_ms": round(m["gate_up_ms"], 4), "down_ms": round(m["down_ms"], 4),
           "flops": flops, "alg_bytes": alg, **_rates(flops, alg, m["ms"])}
    del layer
    torch.cuda.empty_cache()
    return res


def _time_forward(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / steps


def config_finegrained(dev, steps, warmup, tokens=(8, 4096)):
    """Fine-grained shape: hidden 2048, 64 experts, top-6 (renormalised), ffn
    1408, plus 2 shared experts of 1408, through FusedMoE.forward."""
    import torch

    from reframework_amd.moe import FusedMoE

    h, e, k, i, ns = 2048, 64, 6, 1408, 2
    moe = FusedMoE(e, k, h, i, dtype=torch.bfloat16, n_shared_experts=ns).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    with torch.no_grad():
        for prm in moe.parameters():
            prm.copy_(torch.randn(prm.shape, generator=g, device=dev) * 0.02)
    out = {}
    for T in tokens:
        x = (torch.randn(T, h, generator=g, device=dev)).to(torch.bfloat16)
        ms = _time_forward(lambda: moe(x), max(steps, 20), warmup)
        _, ids = moe.route(x)
        n_routed = int(torch.unique(ids).numel())
        flops = 6.0 * T * k * h * i + 2.0 * T * h * e + 6.0 * T * h * i * ns
        alg = (n_routed + ns) * 3 * h * i * 2 + e * h * 2 + 2 * T * h * 2
        out[str(T)] = {"ms": round(ms, 4), "tokens_per_s": round(T / (ms / 1000.0), 1),
                       "routed_experts": n_routed, "flops": flops, "alg_bytes": alg,
                       **_rates(flops, alg, ms)}
    del moe
    torch.cuda.empty_cache()
    return {"workload": "fine-grained moe layer forward (64 routed + 2 shared experts)",
            "hidden": h, "experts": e, "top_k": k, "ffn": i, "shared_experts": ns, "tokens": out}


def _progress(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Staging more than this many pinned pools ended in a host-side segmentation
# fault (exit 139) right after staging, with 32 pools (~129 GiB pinned once
# torch's pinned allocator rounds each 2.8 GB pool up to 4 GiB); the cause is
# not known, so deeper stacks share these pools.
MAX_STAGED_HOST_POOLS = 4


OFFLOAD_MODES = ("max_pack_2_per_layer_lru", "max_pack_2_shared_pool",
                 "max_pack_2_per_layer_lru_cpu_split", "max_pack_2_per_layer_lru_cpu_split_int8",
                 "exact_per_layer_lru_cpu_split", "exact_per_layer_lru_cpu_split_int8",
                 "exact_chunk1_shared_pool", "max_pack_2_shared_pool_t1",
                 "max_pack_2_shared_pool_lookahead_t1")


def config_offload_decode(dev, n_layers, steps, T=8, warmup_steps=4, short_steps=16,
                          modes=OFFLOAD_MODES, host_pools=4):
    """Decode through expert offload: a stack of Mixtral-shape layers (8
    experts each, 352 MB per expert in bf16) whose experts live in pinned host
    memory, with HBM room for 2 experts per layer (64 of 256 expert slots for
    32 layers). Synthetic routing (bypasses the router): per layer and token,
    p=0.7 the previous step's pair again, else two experts from Zipf(1.2).
    Misses stream host->HBM on the caches' copy streams. ``host_pools``
    distinct layers' experts are staged in pinned memory (2.8 GB each); a layer
    l >= host_pools uses layer l mod host_pools's pool (share_host): every
    layer keeps its own routing, HBM slots and LRU, and each miss still copies
    352 MB over PCIe, but only 8 * host_pools distinct experts exist on the
    host.

    Modes (forward, residency), all within 2 HBM slots per layer (the caches
    evict before they copy, so the slots used are the peak resident set,
    reported per mode):
      * max_pack_2_*: the reference's default truncation to RE_MAX_PACK=2
        experts per layer, with (i) a per-layer LRU of 2 or (ii) one LRU over
        (layer, expert) of 2 x layers slots shared by all layers;
      * max_pack_2_per_layer_lru_cpu_split: the same, with the CPU/GPU split
        forward: experts not resident run on the host cores from the pinned
        pool while the GPU runs the others; at most 2 copies in flight bring
        host-computed experts into HBM for later steps;
      * exact_per_layer_lru_cpu_split: every routed expert (no truncation),
        with the CPU/GPU split, ``4 * short_steps`` steps;
      * ..._cpu_split_int8: the same two, the host half on the per-tensor
        int8 bank with the reference's int8 numerics (half the host bytes);
      * exact_chunk1_shared_pool: every routed expert, streamed one expert per
        chunk over the shared pool (chunk i+1's copy runs under chunk i's
        kernels); it moves several times more bytes per step than truncation
        and runs ``short_steps`` steps, named in the key;
      * max_pack_2_shared_pool_t1 and ..._lookahead_t1: batch 1 (a forward
        over more tokens is a prefill to the predictor, as in the reference)
        over a pool with 2 spare slots per layer (4 per layer), without and
        with the lookahead predictor, ``steps // 2`` steps each."""
    import numpy as np
    import torch

    from reframework_amd import _capi, synth
    from reframework_amd.moe import ExpertPool, FusedMoE

    if host_pools > MAX_STAGED_HOST_POOLS:
        raise SystemExit(
            f"--offload-host-pools {host_pools}: at most {MAX_STAGED_HOST_POOLS} staged pinned "
            "pools. 32 staged pools (about 129 GiB pinned after torch rounds each 2.8 GB pool up "
            "to 4 GiB) ended in a host-side segmentation fault right after staging whose cause "
            "is not known; deeper layers share the staged pools instead.")
    h, e, k, i = 4096, 8, 2, 14336
    t_setup = time.perf_counter()
    g = torch.Generator(device=dev).manual_seed(0)
    layers = []
    host_pools = max(1, min(host_pools, n_layers))
    for li in range(n_layers):
        if li < host_pools:
            moe = FusedMoE(e, k, h, i, dtype=torch.bfloat16).to(dev)
            with torch.no_grad():
                for prm in moe.parameters():
                    prm.copy_(torch.randn(prm.shape, generator=g, device=dev) * 0.02)
            moe.build_offload_cache(dev, lru_capacity=2)
        else:
            moe = FusedMoE(e, k, h, i, dtype=torch.bfloat16)
            moe.build_offload_cache(dev, lru_capacity=2, host_from=layers[li % host_pools]._cache)
            moe = moe.to(dev)
        layers.append(moe)
    torch.cuda.synchronize()
    _progress(f"offload decode: {n_layers} layers on {host_pools} pinned host pools "
              f"({time.perf_counter() - t_setup:.0f} s)")
    # peak pinned H2D on this host: one 1 GiB copy through the same entry point
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    cs = torch.cuda.Stream(dev)
    _capi.h2d_async(dst.data_ptr(), src.data_ptr(), n >> 4, cs.cuda_stream)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(cs)
    _capi.h2d_async(dst.data_ptr(), src.data_ptr(), n, cs.cuda_stream)
    b.record(cs)
    b.synchronize()
    peak_h2d = n / (a.elapsed_time(b) / 1000.0) / 1e9
    del src, dst
    expert_bytes = 3 * h * i * 2

    # the host-compute lever: one expert on the host cores from the pinned pool
    # (its pages read once first, as enabling the split does)
    host = layers[0]._cache._host
    layers[0]._cache._host_pool.touch_pages()
    xh = synth.make_tokens(T, h, torch.bfloat16, seed=9)
    host_ms = {}
    for m in (1, 4, T):
        offs = np.array([0, m], np.int32)
        toks = np.arange(m, dtype=np.int32)
        wts = np.ones(m, np.float32)
        out = torch.zeros(T, h)
        times = []
        for rep in range(7):
            ex = rep % e
            t0 = time.perf_counter()
            _capi.host_experts(xh, [host[ex][0]], [host[ex][1]], offs, toks, wts, 0, out)
            times.append(time.perf_counter() - t0)
        host_ms[str(m)] = round(sorted(times[1:])[3] * 1000.0, 3)
    # the same from the int8 bank (half the bytes), built for the split modes anyway
    int8_ms = {}
    if any(m.endswith("_int8") for m in modes):
        layers[0]._cache.quantize_int8_host()
        bank, sums = layers[0]._cache._int8_host, layers[0]._cache._int8_rowsums
        for m in (1, 4, T):
            offs = np.array([0, m], np.int32)
            toks = np.arange(m, dtype=np.int32)
            wts = np.ones(m, np.float32)
            out = torch.zeros(T, h)
            times = []
            for rep in range(7):
                ex = rep % e
                t0 = time.perf_counter()
                _capi.host_experts_int8(xh, [bank[ex][0]], [bank[ex][1]], [bank[ex][2]],
                                        [bank[ex][3]], [sums[ex][0]], [sums[ex][1]], offs, toks,
                                        wts, 0, out)
                times.append(time.perf_counter() - t0)
            int8_ms[str(m)] = round(sorted(times[1:])[3] * 1000.0, 3)
        layers[0]._cache._cpu_split = False
    host_expert = {"tokens_ms": host_ms, "threads": len(os.sched_getaffinity(0)),
                   "gb_s_at_8_tokens": round(expert_bytes / (host_ms[str(T)] / 1000.0) / 1e9, 1),
                   "copy_ms_at_peak_h2d": round(expert_bytes / peak_h2d / 1e6, 3)}
    if int8_ms:
        host_expert["int8_tokens_ms"] = int8_ms
        host_expert["int8_gb_s_at_8_tokens"] = round(
            expert_bytes / 2 / (int8_ms[str(T)] / 1000.0) / 1e9, 1)
    _progress(f"offload decode: host expert {host_ms} ms (int8 {int8_ms} ms), copy "
              f"{host_expert['copy_ms_at_peak_h2d']} ms")

    ids_all, w_all = synth.offload_trace(n_layers, warmup_steps + steps, T, e)
    ids_d = torch.from_numpy(ids_all).to(dev)
    w_d = torch.from_numpy(w_all).to(dev)
    x = (torch.randn(T, h, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    x1 = x[:1].contiguous()

    def run_mode(tag, pool, chunk, n_steps, split=False, lookahead=False, tokens=T, int8=False):
        t_mode = time.perf_counter()
        xin = x if tokens == T else x1

        def fwd(moe, y, st, li):
            wi, ii = w_d[st, li, :tokens], ids_d[st, li, :tokens]
            if split:
                return moe._forward_split(tokens, y, wi, ii, 0)
            if chunk:  # every routed expert, chunk experts at a time
                return moe._forward_streaming(y, wi, ii, 0)
            return moe._forward_offload(tokens, y, wi, ii, 0)

        if chunk:
            os.environ["RE_CHUNK_SIZE"] = str(chunk)
        for moe in layers:
            moe._cache.use_pool(pool)
            moe._cache.log_copies(False)
            moe._predictor = None
            moe._cache._predictor = None
            if split:
                moe._cache.enable_host_experts(int8=int8)
            if lookahead:
                moe.attach_predictor(window=8)
        try:
            for st in range(warmup_steps):
                y = xin
                for li, moe in enumerate(layers):
                    y = fwd(moe, y, st, li)
            torch.cuda.synchronize()
            for moe in layers:
                moe._cache.stats.reset()
                moe._cache.log_copies(True)
            t0 = time.perf_counter()
            for st in range(warmup_steps, warmup_steps + n_steps):
                y = xin
                for li, moe in enumerate(layers):
                    y = fwd(moe, y, st, li)
            torch.cuda.synchronize()
            sec = time.perf_counter() - t0
        finally:
            os.environ.pop("RE_CHUNK_SIZE", None)
            for moe in layers:
                moe._cache._cpu_split = False
        stats = [m._cache.stats for m in layers]
        hits = sum(s_.hits for s_ in stats)
        misses = sum(s_.misses for s_ in stats)
        on_host = sum(s_.host_experts for s_ in stats)
        predicts = sum(s_.predicts for s_ in stats)
        nbytes, copy_ms = 0, 0.0
        for m in layers:
            b_, ms_ = m._cache.copy_summary()
            nbytes += b_
            copy_ms += ms_
        slots = pool.n_slots if pool is not None else sum(m._cache._n_slots for m in layers)
        _progress(f"offload decode: {tag} done ({time.perf_counter() - t_mode:.0f} s)")
        r = {"steps": n_steps, "tokens": tokens, "tokens_per_s": round(tokens * n_steps / sec, 2),
             "ms_per_step": round(sec * 1000.0 / n_steps, 3), "hbm_expert_slots": slots,
             # split: share of the experts run that were resident (the rest ran on
             # the host); otherwise hits / (hits + misses) per OffloadStats
             "hit_rate": round(hits / max(1, hits + (on_host if split else misses)), 4),
             "hits": hits,
             "misses": misses, "lookahead_loads": predicts,
             "h2d_gb_s": round(nbytes / (copy_ms / 1000.0) / 1e9, 2) if copy_ms > 0 else None,
             "h2d_bytes": nbytes, "copy_time_frac": round(copy_ms / 1000.0 / sec, 4)}
        if split:
            r["host_experts"] = on_host
            r["copies"] = misses
        return r

    res = {"workload": f"offload decode, {n_layers} mixtral-shape layers, HBM slots for 2 experts "
                       f"per layer ({2 * n_layers} of {e * n_layers}), host pools of "
                       f"{e * host_pools} distinct experts",
           "layers": n_layers, "tokens": T, "host_pools": host_pools,
           "distinct_host_experts": e * host_pools,
           "peak_pinned_h2d_gb_s": round(peak_h2d, 2), "host_expert": host_expert}
    for mode in modes:
        shared = "shared_pool" in mode
        split = "cpu_split" in mode
        int8 = mode.endswith("_int8")
        t1 = mode.endswith("_t1")
        if mode.startswith("exact_chunk"):
            chunk = int(mode.split("chunk")[1].split("_")[0])
        else:  # the split runs every routed expert when RE_CHUNK_SIZE > 0
            chunk = 8 if mode.startswith("exact") else 0
        pool = ExpertPool(capacity=(4 if t1 else 2) * n_layers) if shared else None
        if chunk:  # every routed expert: several times the bytes of truncation per step
            n_steps = min(steps, 4 * short_steps if split else short_steps)
        else:
            n_steps = max(1, steps // 2) if t1 else steps
        key = f"{mode}_{n_steps}_steps" if n_steps != steps else mode
        res[key] = run_mode(mode, pool, chunk, n_steps, split=split,
                            lookahead=mode.endswith("lookahead_t1"), tokens=1 if t1 else T,
                            int8=int8)
    for moe in layers:
        moe._cache.use_pool(None)
    del layers
    torch.cuda.empty_cache()
    return res


def config_norm_router(dev, steps, warmup, tokens=(1, 16, 4096)):
    """The decoder step before the MoE (residual add + RMSNorm + router, one
    library call) on the Mixtral shape: HBM bound, 4*T*H*2 bytes of rows plus
    the 64 KB gate."""
    import torch

    from reframework_amd import _capi, synth

    h, e, k = 4096, 8, 2
    g = torch.Generator(device=dev).manual_seed(0)
    gate = (torch.randn(e, h, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    nw = (torch.rand(h, generator=g, device=dev) + 0.5).to(torch.bfloat16)
    bias = synth.mixtral_router_bias(e).to(dev)
    out = {}
    for T in tokens:
        x = torch.randn(T, h, generator=g, device=dev).to(torch.bfloat16)
        r = torch.randn(T, h, generator=g, device=dev).to(torch.bfloat16)
        nr, normed = torch.empty_like(x), torch.empty_like(x)
        w = torch.empty(T, k, dtype=torch.float32, device=dev)
        ids = torch.empty(T, k, dtype=torch.int32, device=dev)

        def step():
            _capi.add_rmsnorm_router_topk(x, r, nr, nw, None, 1e-5, gate, bias, k, True, True,
                                          normed, w, ids)

        ms = _time_forward(step, max(steps, 50), warmup)
        alg = 4 * T * h * 2 + e * h * 2
        out[str(T)] = {"us": round(ms * 1000.0, 2), "alg_bytes": alg,
                       "hbm_gb_s": round(alg / (ms / 1000.0) / 1e9, 1),
                       "hbm_frac": round(alg / (ms / 1000.0) / 1e9 / PEAK_HBM_GBS, 4)}
    return {"workload": "residual add + RMSNorm + router top-2, hidden 4096, 8 experts",
            "tokens": out}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE layer runs on a single MI355X; sharding "
              "experts across GPUs is designed but not implemented, so --gpus N > 1 is refused.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    if args.copy_calib:
        src = torch.empty(args.copy_calib, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(max(1, args.steps)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": args.copy_calib, "copies": max(1, args.steps)}))
        return
    layer = Layer(dev)

    if args.profile:
        if args.profile_shape == "finegrained":
            r = config_finegrained(dev, args.steps, args.warmup, tokens=(args.profile,))
            print(json.dumps(r), flush=True)
            return
        if args.profile_shape == "phi35moe":
            from reframework_amd import synth

            del layer
            layer = Layer(dev, hidden=4096, experts=16, top_k=2, ffn=6400,
                          bias=synth.zipf_router_bias(16, 1.1))
        m = measure(layer, args.profile, args.steps, args.warmup)
        print(json.dumps({"tokens": args.profile, "shape": args.profile_shape, **m}), flush=True)
        return

    T = args.tokens
    head = measure(layer, T, args.steps, args.warmup)
    R = T * K
    gemm1_flops = 4.0 * R * H * I
    gemm2_flops = 2.0 * R * H * I
    achieved = gemm1_flops / (head["gate_up_ms"] / 1000.0) / 1e12
    grouped = (gemm1_flops + gemm2_flops) / ((head["gate_up_ms"] + head["down_ms"]) / 1000.0) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": measured_traffic(T),
                "kernel": "ffn_tiled16_kernel<bf16, gate_up>",
                "flops_per_launch": gemm1_flops, "avg_launch_ms": round(head["gate_up_ms"], 4)}

    decode = {}
    for tok in [int(v) for v in args.decode.split(",") if v.strip()]:
        m = measure(layer, tok, max(args.steps, 20), args.warmup)
        n_exp = m["routed_experts"]
        alg_bytes = n_exp * 3 * H * I * 2 + E * H * 2 + 2 * tok * H * 2
        decode[str(tok)] = {
            "ms": round(m["ms"], 4), "tokens_per_s": round(tok / (m["ms"] / 1000.0), 1),
            "routed_experts": n_exp, "alg_bytes": alg_bytes,
            "hbm_gb_s": round(alg_bytes / (m["ms"] / 1000.0) / 1e9, 1),
            "hbm_frac": round(alg_bytes / (m["ms"] / 1000.0) / 1e9 / PEAK_HBM_GBS, 4),
            "gate_up_ms": round(m["gate_up_ms"], 4), "down_ms": round(m["down_ms"], 4),
            "path": m["plan_path"], "down_splits": m["down_splits"],
            "stages": stage_rates(layer, tok, m)}
        if tok == 1:
            decode["1"]["experts_only_same_pair"] = rotating_pairs(
                layer, max(args.steps, 40), args.warmup, rotate=False)
            decode["1"]["experts_only_rotating_pairs"] = rotating_pairs(
                layer, max(args.steps, 40), args.warmup)

    configs = {}
    names = [v.strip() for v in args.configs.split(",") if v.strip()]
    if "phi35moe" in names:
        configs["phi35moe"] = config_phi35moe(dev, max(args.steps // 2, 5), args.warmup)
    if "finegrained" in names:
        configs["finegrained"] = config_finegrained(dev, args.steps, args.warmup)
    if "norm_router" in names:
        configs["norm_router"] = config_norm_router(dev, args.steps, args.warmup)
    if "offload" in names:
        configs["offload_decode"] = config_offload_decode(
            dev, args.offload_layers, args.offload_steps, T=args.offload_tokens,
            host_pools=args.offload_host_pools,
            modes=tuple(m for m in args.offload_modes.split(",") if m) or OFFLOAD_MODES)

    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline(layer, args.cpu_sample_tokens)

    line = {
        "metric": METRIC,
        "value": round(T / (head["ms"] / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "mixtral-8x7b-shape moe layer forward", "tokens": T,
                   "hidden": H, "experts": E, "top_k": K, "ffn": I,
                   "router_bias_sigma": 0.5, "weights_sigma": 0.02},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "grouped_gemm": {"tflops": round(grouped, 2), "mfma_frac": round(grouped / PEAK_BF16_TFLOPS, 4),
                         "gate_up_ms": round(head["gate_up_ms"], 4),
                         "down_ms": round(head["down_ms"], 4)},
        "stages": stage_rates(layer, T, head),
        "decode": decode,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
