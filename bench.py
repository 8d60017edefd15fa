#!/usr/bin/env python3
"""MoE-layer throughput of libzzmoe.so on one MI355X.

Workload: a Gemma-4-shaped q4_0 MoE layer (d=2816,
128 experts, top-8, GeGLU, intermediate 704), S=512 tokens of N(0,1) residuals,
router biased by a seeded Zipf(1.1) per-expert logit offset. A step is one
zz_moe_forward_dev() call on one layer; steps rotate over --layers distinct
layers (default 30, ~12.8 GB of experts) so the weights cannot sit in the 256 MB
MALL. Inputs and weights are resident in HBM before timing starts. The other
configs are reported under their own keys:
  decode   configs[0], the same layers at S=1;
  lfm      configs[2], LFM2.5-shaped (d=2048, 32 experts, top-4 sigmoid, SwiGLU 1792,
           gate/up q4_0, down q8_0) at S=1, 8 and 256;
  maple    configs[3], Maple-shaped tq2 (d=2048, 256 experts, top-8, SwiGLU 768,
           P(0)=0.4 ternary codes, one f32 alpha per row as tq2.h lays it out) at
           S=1 and 512;
  stack    configs[4], the 30-layer stack (each MoE layer with gemma's dense MLP and
           layer combine, a tied q4_0 head of 262144 rows, 512-token prefill then 256
           greedy decode steps, attention as the identity).

Also reported: per-kernel durations from HIP events recorded by the library on
the stream each kernel runs on (zz_moe_profile), the roofline of each leg's
dominant kernel, and the reference's own OpenMP CPU path (gemma4.c's moe_start +
moe_finish compiled from its sources into oracle/_ref) timed on this host, in a
child process pinned as OMP_PROC_BIND=close / OMP_PLACES=cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import statistics
import subprocess
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_PEAK_TOPS = 5000.0        # MI355X dense int8 matrix-core peak (5.0 POP/s)
D, MI, E, K = 2816, 704, 128, 8


def tensor_bytes(fmt, O, I):
    """q40.h:313-314, 461-462; tq2.h:81-86."""
    if fmt == 1:
        return O * (I // 32) * 18
    if fmt == 2:
        return O * (I // 32) * 34
    return O * 4 + O * (I // 4)


Q40_TENSOR = lambda O, I: tensor_bytes(1, O, I)   # noqa: E731
GATE_B = Q40_TENSOR(MI, D)
DOWN_B = Q40_TENSOR(D, MI)
REC_B = 2 * GATE_B + DOWN_B

# the layer shapes of BASELINE.json's configs; gating / activation codes of zz_moe.h
CONFIGS = {
    "gemma": dict(D=2816, MI=704, E=128, K=8, gating=0, act=0, fmts=(1, 1, 1)),
    "lfm": dict(D=2048, MI=1792, E=32, K=4, gating=1, act=1, fmts=(1, 1, 2)),
    "maple": dict(D=2048, MI=768, E=256, K=8, gating=2, act=2, fmts=(3, 3, 3)),
}


def rec_bytes(c):
    return (tensor_bytes(c["fmts"][0], c["MI"], c["D"]) + tensor_bytes(c["fmts"][1], c["MI"], c["D"])
            + tensor_bytes(c["fmts"][2], c["D"], c["MI"]))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(leg, kernel):
    """HBM bytes per launch of `kernel` in leg `leg` (e.g. gemma512) from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by a known-size copy), or None
    where that leg was not measured."""
    p = os.path.join(HERE, "profiles", "ffn_traffic.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        f = line.split()
        if len(f) == 4 and f[0] == "traffic_bytes_per_launch" and f[1] == leg and f[2] == kernel:
            return float(f[3])
    return None


def measured_mfma_busy(leg, kernel):
    """Fraction of the matrix cores' cycles busy in `kernel` of leg `leg` (e.g.
    gemma512) from the committed SQ_VALU_MFMA_BUSY_CYCLES summary, or None where that
    leg was not measured."""
    p = os.path.join(HERE, "profiles", "ffn_mfma_gemma_s512_counters.md")
    if not os.path.exists(p):
        return None
    for line in open(p):
        f = line.split()
        if len(f) == 4 and f[0] == "mfma_busy_frac" and f[1] == leg and f[2] == kernel:
            return float(f[3])
    return None


def zipf_offsets(rng, n):
    """-1.1 ln(rank) for a seeded permutation of ranks 1..n (the config 2 router skew)."""
    return (-1.1 * np.log(rng.permutation(n) + 1)).astype(np.float32)


def build_layers(zz, torch, n_layers, seed):
    """n_layers Gemma layers. Experts: N(0, 0.02) weights drawn on the device and
    quantised by zz_quantize (bit-exact q40_quant_row); router/norms on the host."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device="cuda")
    layers, host = [], []
    per = 3 * MI * D                                       # f32 values per expert
    chunk = 16                                             # experts per generation pass
    buf_f = torch.empty(chunk * per, dtype=torch.float32, device="cuda")
    buf_q = torch.empty(chunk * REC_B, dtype=torch.uint8, device="cuda")
    for li in range(n_layers):
        router = rng.standard_normal((E, D), dtype=np.float32)
        rscale = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        pes = (1 + 0.1 * rng.random(E)).astype(np.float32)
        pre = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        post = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        zipf = zipf_offsets(rng, E)
        m = zz.MoeLayer(D, MI, E, K, zz.ZZ_GATE_SOFTMAX_PES, zz.ZZ_ACT_GEGLU_TANH,
                        (1, 1, 1), router, rscale, pes, zipf, pre, post, use_bias=1, eps=1e-6)
        gen.manual_seed(seed * 1000 + li)
        for e0 in range(0, E, chunk):
            buf_f.normal_(0.0, 0.02, generator=gen)
            zz.quantize_dev(1, buf_f.data_ptr(), buf_q.data_ptr(), buf_f.numel(),
                            torch.cuda.current_stream().cuda_stream)
            torch.cuda.current_stream().synchronize()
            for j in range(chunk):
                m.upload_dev(e0 + j, buf_q.data_ptr() + j * REC_B, REC_B)
        layers.append(m)
        host.append(dict(router=router, rscale=rscale, pes=pes, pre=pre, post=post, zipf=zipf))
    del buf_f, buf_q
    torch.cuda.empty_cache()
    return layers, host


def layer_experts_host(zz, torch, seed, li, ids=None):
    """Gemma layer li's expert records regenerated on the device, copied to the host
    (only experts `ids` when given; the others stay zero)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed * 1000 + li)
    per, chunk = 3 * MI * D, 16
    out = np.zeros(E * REC_B, np.uint8)
    want = set(range(E)) if ids is None else {int(e) for e in ids}
    buf_f = torch.empty(chunk * per, dtype=torch.float32, device="cuda")
    buf_q = torch.empty(chunk * REC_B, dtype=torch.uint8, device="cuda")
    for e0 in range(0, E, chunk):
        buf_f.normal_(0.0, 0.02, generator=gen)
        zz.quantize_dev(1, buf_f.data_ptr(), buf_q.data_ptr(), buf_f.numel(),
                        torch.cuda.current_stream().cuda_stream)
        torch.cuda.current_stream().synchronize()
        if want >= set(range(e0, e0 + chunk)):
            out[e0 * REC_B:(e0 + chunk) * REC_B] = buf_q.cpu().numpy()
        else:
            for e in sorted(want & set(range(e0, e0 + chunk))):
                out[e * REC_B:(e + 1) * REC_B] = buf_q[(e - e0) * REC_B:(e - e0 + 1) * REC_B].cpu().numpy()
    return out


def tq2_dev(torch, O, I, gen):
    """One tq2 tensor (tq2.h:17-28: alpha[O] f32, then code rows) on the device:
    codes 0/1/2 (-1/0/+1) with P(0) = 0.4, packed as tq2.h:46-51 (code j in byte
    j % 16 of its 64-group at bit 2 ((j / 16) % 4)); alpha near the absmean of
    N(0, 0.02) weights."""
    u = torch.rand(O, I, generator=gen, device="cuda")
    c = torch.ones(O, I, dtype=torch.uint8, device="cuda")
    c[u < 0.3] = 0
    c[u >= 0.7] = 2
    c = c.view(O, I // 64, 4, 16)
    packed = c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6)
    alpha = (0.016 * (1 + 0.05 * torch.randn(O, generator=gen, device="cuda"))).float()
    return torch.cat([alpha.view(torch.uint8), packed.reshape(-1)])


def build_cfg_layers(zz, torch, name, n_layers, seed):
    """n_layers LFM- or Maple-shaped layers, experts generated on the device.
    LFM: N(0, 0.02) weights, gate/up quantised to q4_0 and down to q8_0 by
    zz_quantize; router N(0, 1) rows and N(0, 0.1) biases (lfm25.c:636-668).
    Maple: tq2 tensors from tq2_dev; router N(0, 1) rows (maple.c:582-601)."""
    c = CONFIGS[name]
    Dc, MIc, Ec, Kc = c["D"], c["MI"], c["E"], c["K"]
    rb = rec_bytes(c)
    rng = np.random.default_rng(seed + 17)
    gen = torch.Generator(device="cuda")
    st = torch.cuda.current_stream()
    layers = []
    for li in range(n_layers):
        router = rng.standard_normal((Ec, Dc), dtype=np.float32)
        if name == "lfm":
            bias = (0.1 * rng.standard_normal(Ec)).astype(np.float32)
            m = zz.MoeLayer(Dc, MIc, Ec, Kc, zz.ZZ_GATE_SIGMOID_BIAS, zz.ZZ_ACT_SWIGLU, c["fmts"],
                            router, bias=bias, norm_topk=1, use_bias=1, routed_scaling=1.0)
        else:
            m = zz.MoeLayer(Dc, MIc, Ec, Kc, zz.ZZ_GATE_SOFTMAX_TOPK, zz.ZZ_ACT_SWIGLU_CLAMP,
                            c["fmts"], router, norm_topk=1, clamp=7.0)
        if m.record_bytes != rb:
            raise RuntimeError(f"{name}: record {m.record_bytes} B, expected {rb}")
        gen.manual_seed(seed * 1000 + 500 + li)
        if name == "lfm":
            gu = torch.empty(2 * MIc * Dc, dtype=torch.float32, device="cuda")
            dn = torch.empty(Dc * MIc, dtype=torch.float32, device="cuda")
            rec = torch.empty(rb, dtype=torch.uint8, device="cuda")
            nq = 2 * tensor_bytes(1, MIc, Dc)
            for e in range(Ec):
                gu.normal_(0.0, 0.02, generator=gen)
                dn.normal_(0.0, 0.02, generator=gen)
                zz.quantize_dev(1, gu.data_ptr(), rec.data_ptr(), gu.numel(), st.cuda_stream)
                zz.quantize_dev(2, dn.data_ptr(), rec.data_ptr() + nq, dn.numel(), st.cuda_stream)
                st.synchronize()
                m.upload_dev(e, rec.data_ptr(), rb)
        else:
            for e in range(Ec):
                rec = torch.cat([tq2_dev(torch, MIc, Dc, gen), tq2_dev(torch, MIc, Dc, gen),
                                 tq2_dev(torch, Dc, MIc, gen)])
                st.synchronize()
                m.upload_dev(e, rec.data_ptr(), rb)
        layers.append(m)
    torch.cuda.empty_cache()
    return layers


PREWARM_S = 0.2


def time_steps(torch, layers, xs, out, S, steps, warmup):
    st = torch.cuda.current_stream()
    L = len(layers)
    # every rotated layer runs once before the timed loop, whatever `warmup` is: a
    # layer's first forward at a batch size sizes its workspace (hipMalloc and two
    # stream synchronisations), which must not fall between the timing events
    for i, m in enumerate(layers):
        m.forward_dev(xs[i % len(xs)].data_ptr(), out.data_ptr(), S, stream=st.cuda_stream)
    # then PREWARM_S seconds of untimed steps: on a GPU that was idle the first tens of
    # milliseconds of load run a few percent slower (the same 20 timed steps took 228 us
    # after 5 warm-up steps, 216 us after 200), which is not the steady state
    t_end, i = time.perf_counter() + PREWARM_S, 0
    while time.perf_counter() < t_end:
        for _ in range(L):
            layers[i % L].forward_dev(xs[i % len(xs)].data_ptr(), out.data_ptr(), S, stream=st.cuda_stream)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        layers[i % L].forward_dev(xs[i % len(xs)].data_ptr(), out.data_ptr(), S,
                                  stream=st.cuda_stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        layers[i % L].forward_dev(xs[i % len(xs)].data_ptr(), out.data_ptr(), S,
                                  stream=st.cuda_stream)
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, e0.elapsed_time(e1) / 1e3


def kernel_profile(zz, torch, layers, xs, out, S, K_):
    """One profiled pass over every layer: per-kernel mean duration (HIP events on
    the launch stream) and the routing of each step for the byte accounting."""
    st = torch.cuda.current_stream()
    eidx = [torch.empty(S * K_, dtype=torch.int32, device="cuda") for _ in layers]
    zz.profile(True)
    for i, m in enumerate(layers):
        m.forward_dev(xs[i % len(xs)].data_ptr(), out.data_ptr(), S,
                      d_eidx=eidx[i].data_ptr(), stream=st.cuda_stream)
    torch.cuda.synchronize()
    prof = zz.profile_read()
    zz.profile(False)
    nus = [len(np.unique(e.cpu().numpy())) for e in eidx]
    return prof, nus


def algorithmic_bytes(c, S, nu):
    """Per-kernel and whole-layer HBM bytes, each distinct byte counted once: the
    union's expert tensors, the activations the kernel reads and writes (int8 codes
    plus per-block scale and sum for the quantised input and hidden, f32 partials
    y[S*K, D] between the down and combine kernels), router, norms and the layer's
    f32 input and output."""
    Dc, MIc, Ec, Kc, f = c["D"], c["MI"], c["E"], c["K"], c["fmts"]
    g, u, d = tensor_bytes(f[0], MIc, Dc), tensor_bytes(f[1], MIc, Dc), tensor_bytes(f[2], Dc, MIc)
    P = S * Kc
    xq = S * Dc + S * (Dc // 32) * 8
    h = P * MIc + P * (MIc // 32) * 8
    y = P * Dc * 4
    up = nu * (g + u) + xq + h
    down = nu * d + h + y
    layer = nu * (g + u + d) + Ec * Dc * 4 + 3 * Dc * 4 + Ec * 8 + 2 * S * Dc * 4
    return dict(ffn_up=up, ffn_down=down, dec_down=down, layer=layer)


def run_leg(zz, torch, name, layers, S, steps, warmup, seed):
    """Time `steps` forwards at S tokens rotating over `layers`, profile one pass,
    and return the leg's figures with the roofline of its dominant kernel."""
    c = CONFIGS[name]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + S)
    xs = [torch.randn(S, c["D"], generator=g, device="cuda") for _ in range(4)]
    out = torch.empty(S, c["D"], device="cuda")
    wall, ev = time_steps(torch, layers, xs, out, S, steps, warmup)
    prof, nus = kernel_profile(zz, torch, layers, xs, out, S, c["K"])
    nu = float(np.mean(nus))
    by = algorithmic_bytes(c, S, nu)
    kern = {k: (ms / n * 1e3 if n else 0.0) for k, (ms, n) in prof.items() if n}   # us / launch
    step = ev / steps
    dom = max((k for k in ("ffn_up", "ffn_down", "dec_down") if k in kern), key=lambda k: kern[k])
    ach = by[dom] / (kern[dom] * 1e-6) / 1e9
    log(f"{name} S={S}: {steps} steps wall {wall * 1e3:.2f} ms events {ev * 1e3:.2f} ms "
        f"-> {step * 1e6:.1f} us/step, nu {nu:.1f}; kernels (us): "
        + ", ".join(f"{k} {v:.1f}" for k, v in kern.items()))
    return dict(tokens=S, steps=steps, us_per_step=step * 1e6, tokens_per_s=S / step,
                wall_us_per_step=wall / steps * 1e6, mean_union_experts=nu, kernels_us=kern,
                roofline={"bound": "hbm", "kernel": dom, "achieved": ach, "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": ach / HBM_PEAK_GBS,
                          "traffic": measured_traffic(f"{name}{S}", dom), "algorithmic_bytes": by[dom],
                          "kernel_us": kern[dom]},
                layer_roofline={"bound": "hbm", "algorithmic_bytes": by["layer"],
                                "achieved": by["layer"] / step / 1e9,
                                "frac": by["layer"] / step / 1e9 / HBM_PEAK_GBS},
                mfma=mfma_use(c, S, kern, f"{name}{S}"))


def mfma_use(c, S, kern, leg):
    """int8 matrix-core use of the batched FFN kernels (absent on the decode path):
    the useful int8 operations (2 per multiply-add of the routed pairs' gate, up and
    down products, padding excluded) per kernel second against the dense int8 peak,
    and the busy fraction read by rocprofv3 where the counters were taken."""
    if kern.get("dec_down"):                     # decode: dot4 GEMV kernels, no matrix cores
        return None
    P, D, MI = S * c["K"], c["D"], c["MI"]
    ops = {"ffn_up": 2.0 * P * 2 * MI * D, "ffn_down": 2.0 * P * D * MI}
    out = {}
    for k, n in ops.items():
        if kern.get(k):
            a = n / (kern[k] * 1e-6) / 1e12
            out[k] = {"achieved": a, "peak": MFMA_PEAK_TOPS, "unit": "TOP/s", "frac": a / MFMA_PEAK_TOPS,
                      "int8_ops": n, "kernel_us": kern[k], "busy": measured_mfma_busy(leg, k)}
    return out or None


# ------------------------------------------------------------------ CPU baseline
def host_cores():
    """Physical cores of one socket that this process may run on (lscpu's CPU,
    CORE, SOCKET table against the affinity mask), the socket's full count, and
    the affinity size."""
    allowed = os.sched_getaffinity(0)
    try:
        txt = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True, text=True,
                             timeout=30).stdout
        rows = [tuple(int(v) for v in ln.split(",")[:3]) for ln in txt.splitlines()
                if ln and not ln.startswith("#")]
    except (OSError, ValueError, subprocess.SubprocessError):
        rows = []
    if not rows:
        return len(allowed), len(allowed), len(allowed)
    per_socket = {}
    for cpu, core, sock in rows:
        per_socket.setdefault(sock, [set(), set()])
        per_socket[sock][0].add(core)
        if cpu in allowed:
            per_socket[sock][1].add(core)
    sock = max(per_socket, key=lambda s: len(per_socket[s][1]))
    return len(per_socket[sock][1]), len(per_socket[sock][0]), len(allowed)


def cpu_layers_dir(zz, torch, host, seed, n_layers):
    """Write the first n_layers Gemma layers for the CPU child: each layer's expert
    records (regenerated exactly as uploaded) and router tensors, in a directory
    under /dev/shm where present. The Zipf skew the GPU gets from its logit bias
    is given to the unmodified reference router through input column 0: every row
    has x[0] = 1, and router column 0 holds zipf * sqrt(D) / router_scale[0], so
    with rms(x) ~ 1 each logit gains ~zipf_e (gemma4.c:589-600)."""
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    d = tempfile.mkdtemp(prefix="zzbench_", dir=base)
    for li in range(n_layers):
        h = host[li]
        router = h["router"].copy()
        router[:, 0] = h["zipf"] * np.float32(np.sqrt(D)) / h["rscale"][0]
        np.savez(os.path.join(d, f"layer{li}.npz"), router=router, rscale=h["rscale"], pes=h["pes"],
                 pre=h["pre"], post=h["post"])
        layer_experts_host(zz, torch, seed, li).tofile(os.path.join(d, f"experts{li}.bin"))
    return d


def cpu_child(argv):
    """Runs in a child process started with OMP_NUM_THREADS / OMP_PROC_BIND=close /
    OMP_PLACES=cores, so that the reference's OpenMP team is pinned from its first
    region. Times gemma4.c's moe_start + moe_finish (oracle/_ref) at S=1 and S=512 at
    the given thread counts: 3 warm-ups, then the median of the reps, rotating over
    the layers. Prints one JSON line."""
    import ctypes as C
    ap = argparse.ArgumentParser()
    ap.add_argument("--dir")
    ap.add_argument("--layers", type=int)
    ap.add_argument("--threads", type=str)
    ap.add_argument("--seed", type=int)
    a = ap.parse_args(argv)
    sys.path.insert(0, os.path.join(HERE, "tests"))
    import zzref as Z
    ref = Z.ref_lib("gemma4")
    kern = Z.ref_lib("kernels")
    if ref is None:
        print(json.dumps({"error": "oracle/_ref not built"}), flush=True)
        return
    f32p = C.POINTER(C.c_float)
    ref.ref_g4_layer_new.restype = C.c_void_p
    ref.ref_g4_layer_new.argtypes = [C.c_int] * 4 + [C.c_float] + [f32p] * 5 + [C.c_void_p, C.c_int64, C.c_int]
    ref.ref_g4_layer_call.argtypes = [C.c_void_p, f32p, C.c_int, f32p, C.POINTER(C.c_int)]
    ref.ref_g4_layer_free.argtypes = [C.c_void_p]
    variant = {2: "AVX2", 1: "NEON", 0: "scalar"}.get(kern.ref_simd_variant() if kern else -1, "unknown")
    keep, handles = [], []
    for li in range(a.layers):
        z = np.load(os.path.join(a.dir, f"layer{li}.npz"))
        w = [np.ascontiguousarray(z[k]) for k in ("router", "rscale", "pes", "pre", "post")]
        ex = np.fromfile(os.path.join(a.dir, f"experts{li}.bin"), np.uint8)
        keep.append((w, ex))
        h = ref.ref_g4_layer_new(D, MI, E, K, 1e-6, *(Z.ptr(v) for v in w),
                                 C.c_void_p(ex.ctypes.data), REC_B, 512)
        if not h:
            raise RuntimeError("ref_g4_layer_new failed")
        handles.append(h)
    rng = np.random.default_rng(a.seed + 7)
    res = {"variant": variant, "layers": a.layers}
    nu = C.c_int()
    for nth in (int(t) for t in a.threads.split(",")):
        ref.ref_g4_set_threads(nth)
        for S, reps in ((1, 200), (512, 20 if nth > 2 else 10)):
            x = rng.standard_normal((S, D), dtype=np.float32)
            x[:, 0] = 1.0
            out = np.zeros((S, D), np.float32)
            times, nus = [], []
            for i in range(3 + reps):
                t0 = time.perf_counter()
                ref.ref_g4_layer_call(handles[i % a.layers], Z.ptr(x), S, Z.ptr(out), C.byref(nu))
                dt = time.perf_counter() - t0
                if i >= 3:
                    times.append(dt)
                    nus.append(nu.value)
            med = statistics.median(times)
            res[f"t{nth}_s{S}"] = dict(threads=nth, tokens=S, reps=reps, median_ms=med * 1e3,
                                       tokens_per_s=S / med, mean_union_experts=float(np.mean(nus)))
    for h in handles:
        ref.ref_g4_layer_free(h)
    print(json.dumps(res), flush=True)


def cpu_baseline(zz, torch, host, seed, n_layers):
    """The reference's own moe_start + moe_finish on this host, in a pinned child
    process: all physical cores of one socket (within this process's affinity) and
    the reference's default of 2 threads, at S=512 and S=1."""
    cores, socket_cores, affinity = host_cores()
    d = cpu_layers_dir(zz, torch, host, seed, n_layers)
    try:
        env = dict(os.environ, OMP_NUM_THREADS=str(cores), OMP_PROC_BIND="close", OMP_PLACES="cores")
        p = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", "--dir", d,
                            "--layers", str(n_layers), "--threads", f"{cores},2", "--seed", str(seed)],
                           env=env, capture_output=True, text=True, timeout=900)
    finally:
        for f in os.listdir(d):
            os.unlink(os.path.join(d, f))
        os.rmdir(d)
    if p.returncode != 0:
        log(p.stderr[-2000:])
        raise RuntimeError(f"CPU baseline child failed ({p.returncode})")
    r = json.loads(p.stdout.strip().splitlines()[-1])
    if "error" in r:
        return None
    main_ = r[f"t{cores}_s512"]
    return dict(value=main_["tokens_per_s"], unit="tokens/s", cores=cores, kind="reference",
                variant=r["variant"],
                sample=f"gemma4.c moe_start+moe_finish (oracle/_ref, {r['variant']} OpenMP, built "
                       f"gcc -O3 -march=x86-64-v3 -mavx2 -mfma -fopenmp: the reference's AVX2 kernel "
                       f"path; its own Makefile's -march=native takes the same path), S=512, "
                       f"median of {main_['reps']} calls after 3 warm-ups, rotating over "
                       f"{n_layers} layers' experts preloaded in RAM; Zipf(1.1) routing via "
                       f"input column 0 (mean union {main_['mean_union_experts']:.1f} experts)",
                host=dict(socket_physical_cores=socket_cores, affinity_cpus=affinity,
                          omp="OMP_PROC_BIND=close OMP_PLACES=cores"),
                s512=main_, s1=r[f"t{cores}_s1"], threads2=dict(s512=r["t2_s512"], s1=r["t2_s1"]))


DI, V = 2112, 262144                     # Gemma-4 dense_inter and vocabulary
DENSE_B = 2 * Q40_TENSOR(DI, D) + Q40_TENSOR(D, DI)
TABLE_B = Q40_TENSOR(V, D)


def device_q40(zz, torch, n, gen, sigma=0.02):
    """n N(0, sigma) weights quantised to q4_0 on the device (bit-exact
    q40_quant_row), as a uint8 tensor in the reference layout."""
    f = torch.empty(n, dtype=torch.float32, device="cuda")
    f.normal_(0.0, sigma, generator=gen)
    q = torch.empty(n // 32 * 18, dtype=torch.uint8, device="cuda")
    zz.quantize_dev(1, f.data_ptr(), q.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().synchronize()
    return q


def flash_tensors(zz, torch, table, seed, cluster_size=32, probe_fraction=512 / 4748, n_force=2):
    """A synthetic FlashHead for the tied table in tools/flashhead.py's shapes: V/32
    balanced clusters (a seeded permutation of the ids), the probe count at the
    builder's default fraction, each centroid the q4_0 of its members' mean row
    (dequantised and averaged on the device). Arguments for Head.flash."""
    Vt = table.shape[0] // (18 * (D // 32))
    nc = Vt // cluster_size
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 4748)
    perm = torch.randperm(Vt, generator=g, device="cuda")
    cent = torch.empty(nc, D, dtype=torch.float32, device="cuda")
    t = torch.from_numpy(table).cuda().view(Vt, D // 32, 18)
    for c0 in range(0, nc, 1024):                 # 1024 clusters (32768 rows) per pass
        ids = perm[c0 * cluster_size:(c0 + 1024) * cluster_size]
        blk = t[ids]
        dsc = blk[:, :, :2].contiguous().view(torch.float16).float()
        q = blk[:, :, 2:]
        w = (torch.cat([q & 15, q >> 4], dim=2).float() - 8.0) * dsc
        cent[c0:c0 + 1024] = w.view(-1, cluster_size, D).mean(1)
    del t
    cq = torch.empty(nc * (D // 32) * 18, dtype=torch.uint8, device="cuda")
    zz.quantize_dev(zz.GPU_FMT_Q40, cent.data_ptr(), cq.data_ptr(), nc * D, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    tmap = perm.view(nc, cluster_size).to(torch.int32).cpu().numpy()
    n_probes = max(1, int(round(nc * probe_fraction)))
    return (cq.cpu().numpy(), nc, tmap, cluster_size, n_probes, np.ones(nc, np.float32), 1,
            np.arange(1, 1 + n_force, dtype=np.int32))


def build_stack(zz, torch, layers, seed, flash=True, keep_host=False):
    """BASELINE config 5 around the MoE layers `layers`: per layer a q4_0 dense MLP
    (dense_inter 2112) and the layer combine (gemma4.c:1003-1030), under a tied q4_0
    embedding / lm_head of Gemma-4's 262144 rows; attention is the identity. Returns
    a dict: blocks, head, stack, objs (to close), flash (Head.flash arguments, or
    None), and with keep_host the dense branches' host weights per layer (mlp,
    pre_ffn_ln, post_ffn_ln1, post_ffn_ln, layer_scalar) for a CPU check."""
    rng = np.random.default_rng(seed + 500)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed * 7919)
    objs, blocks, dense = [], [], []
    for li, m in enumerate(layers):
        pre = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        post1 = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        d = zz.MoeLayer(D, DI, 1, 1, zz.ZZ_GATE_DENSE, zz.ZZ_ACT_GEGLU_TANH, (1, 1, 1), None,
                        pre_ln=pre, post_ln=post1, eps=1e-6)
        q = device_q40(zz, torch, 3 * DI * D, gen)
        d.upload_dev(0, q.data_ptr(), DENSE_B)
        post = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        scalar = float(np.float32(0.5 + 0.5 * rng.random()))
        if keep_host:
            dense.append(dict(mlp=q.cpu().numpy(), pre_ffn_ln=pre, post_ffn_ln1=post1,
                              post_ffn_ln=post, layer_scalar=scalar))
        del q
        b = zz.FfnBlock(m, d, post, scalar)
        objs += [b, d]
        blocks.append(b)
    parts = []
    for r0 in range(0, V, 16384):                        # 16384 rows per pass: 185 MB of f32
        parts.append(device_q40(zz, torch, 16384 * D, gen).cpu().numpy())
    table = np.concatenate(parts)
    del parts
    torch.cuda.empty_cache()
    fnorm = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    head = zz.Head(table, V, D, fnorm, 1e-6, float(np.sqrt(np.float32(D))), 30.0)
    fl = flash_tensors(zz, torch, table, seed) if flash else None
    stack = zz.Stack(blocks, head)
    objs += [stack, head]
    return dict(blocks=blocks, head=head, stack=stack, objs=objs, flash=fl, dense=dense,
                table=table if keep_host else None, fnorm=fnorm)


def stack_bench(zz, torch, layers, seed, prefill_S, steps):
    """BASELINE config 5 (build_stack): a prefill of prefill_S N(0,1) rows, then
    greedy decode steps whose token ids stay on the device, both timed with HIP
    events on the launching stream."""
    c5 = build_stack(zz, torch, layers, seed)
    stack, head, flash, objs = c5["stack"], c5["head"], c5["flash"], c5["objs"]
    st = torch.cuda.current_stream()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 99)
    H0 = torch.randn(prefill_S, D, generator=g, device="cuda")
    H = H0.clone()
    tok = torch.zeros(steps + 1, dtype=torch.int32, device="cuda")
    stack.prefill_dev(H.data_ptr(), prefill_S, tok.data_ptr(), st.cuda_stream)   # warm-up
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 3
    e0.record(st)
    for _ in range(reps):
        H.copy_(H0)
        stack.prefill_dev(H.data_ptr(), prefill_S, tok.data_ptr(), st.cuda_stream)
    e1.record(st)
    torch.cuda.synchronize()
    copy_ms = prefill_S * D * 4 * 2 / 4e12 * 1e3                      # the H reset, ~3 us
    prefill_s = (e0.elapsed_time(e1) / reps - copy_ms) / 1e3
    out = {}
    for graph in (False, True):
        stack.decode_dev(tok.data_ptr(), 4, graph=graph, stream=st.cuda_stream)     # warm / capture
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(st)
        stack.decode_dev(tok.data_ptr(), steps, graph=graph, stream=st.cuda_stream)
        e1.record(st)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        out["graph" if graph else "eager"] = dict(tokens_per_s=steps / (e0.elapsed_time(e1) / 1e3),
                                                  ms_per_token=e0.elapsed_time(e1) / steps,
                                                  host_wall_ms_per_token=wall * 1e3 / steps)
    toks = tok.cpu().numpy()
    # the same decode with FlashHead (gemma4.c:1055-1110) in place of the full head
    head.flash(*flash)
    stack.use_flash(True)
    fl = {}
    for graph in (False, True):
        stack.decode_dev(tok.data_ptr(), 4, graph=graph, stream=st.cuda_stream)     # warm / capture
        torch.cuda.synchronize()
        e0.record(st)
        stack.decode_dev(tok.data_ptr(), steps, graph=graph, stream=st.cuda_stream)
        e1.record(st)
        torch.cuda.synchronize()
        fl["graph" if graph else "eager"] = dict(tokens_per_s=steps / (e0.elapsed_time(e1) / 1e3),
                                                 ms_per_token=e0.elapsed_time(e1) / steps)
    # algorithmic bytes of one decode token: per layer the 8 routed experts, the
    # router, the dense MLP and the norm vectors; the head table once (FlashHead: the
    # centroids and the probed rows)
    per_layer = K * REC_B + E * D * 4 + DENSE_B + 8 * D * 4
    step_bytes = len(layers) * per_layer + TABLE_B + D * 4
    NC, CS, NP, nforce = flash[1], flash[3], flash[4], len(flash[7])
    flash_bytes = len(layers) * per_layer + Q40_TENSOR(NC, D) + Q40_TENSOR(NP * CS + nforce, D) + D * 4
    fbest = max(fl.values(), key=lambda v: v["tokens_per_s"])
    best = max(out.values(), key=lambda v: v["tokens_per_s"])
    for o in objs:
        o.close()
    return dict(
        workload=f"gemma4 stack: {len(layers)} layers x (MoE E={E} top-{K} MI={MI} + dense "
                 f"MLP {DI}) q4_0, tied q4_0 head V={V}, attention = identity",
        prefill=dict(tokens=prefill_S, ms=prefill_s * 1e3, tokens_per_s=prefill_S / prefill_s),
        decode=dict(steps=steps, eager=out["eager"], graph=out["graph"],
                    tokens_per_s=best["tokens_per_s"], hbm_bytes_per_token=step_bytes,
                    hbm_GBs=step_bytes * best["tokens_per_s"] / 1e9,
                    hbm_frac=step_bytes * best["tokens_per_s"] / 1e9 / HBM_PEAK_GBS,
                    distinct_tokens=int(len(np.unique(toks))), first_tokens=toks[:12].tolist()),
        flash_decode=dict(head=f"FlashHead: {NC} balanced clusters of {CS} (random permutation, "
                               f"centroids the q4_0 member means), {NP} probed, {nforce} forced",
                          eager=fl["eager"], graph=fl["graph"], tokens_per_s=fbest["tokens_per_s"],
                          hbm_bytes_per_token=flash_bytes,
                          hbm_GBs=flash_bytes * fbest["tokens_per_s"] / 1e9,
                          hbm_frac=flash_bytes * fbest["tokens_per_s"] / 1e9 / HBM_PEAK_GBS))


def main():
    if "--cpu-child" in sys.argv:
        cpu_child([a for a in sys.argv[1:] if a != "--cpu-child"])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--cfg-layers", type=int, default=12,
                    help="layers rotated in the lfm / maple legs (~3 GB of experts each)")
    ap.add_argument("--tokens", type=int, default=512)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--legs", default="gemma,lfm,maple",
                    help="comma list of gemma / lfm / maple, or name:S for one size (lfm:256)")
    ap.add_argument("--cpu-layers", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the 30-layer stack (config 5)")
    ap.add_argument("--stack-steps", type=int, default=256)
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="only run one plain device-to-device copy of this many MiB (the "
                         "known-size kernel that scales FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only: the MoE layer is measured on a single "
              "MI355X (expert-parallel sharding across GPUs is designed, not built).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calib_copy_mb:
        n = args.calib_copy_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty(n, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {n} bytes device to device")
        return
    sizes = {"gemma": [args.tokens, 1], "lfm": [1, 8, 256], "maple": [1, 512]}
    legs = {}
    for item in args.legs.split(","):
        name, _, S = item.partition(":")
        legs.setdefault(name, []).extend([int(S)] if S else sizes[name])
    import zunzuncito_amd as zz
    name = zz.init()
    log("device:", name)
    # a stream of our own: handle 0 would mean "the library's stream" to the ABI
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)

    def steps_for(S):
        return args.steps * 4 if S == 1 else args.steps * 2 if S <= 8 else args.steps

    res, layers, host = {}, None, None
    for leg, Ss in legs.items():
        t0 = time.time()
        if leg == "gemma":
            layers, host = build_layers(zz, torch, args.layers, args.seed)
            ls = layers
        else:
            ls = build_cfg_layers(zz, torch, leg, args.cfg_layers, args.seed)
        log(f"built {len(ls)} {leg} layers ({len(ls) * rec_bytes(CONFIGS[leg]) * CONFIGS[leg]['E'] / 1e9:.1f} "
            f"GB experts) in {time.time() - t0:.1f}s")
        res[leg] = {S: run_leg(zz, torch, leg, ls, S, steps_for(S), args.warmup, args.seed) for S in Ss}
        if leg != "gemma":
            for m in ls:
                m.close()
            torch.cuda.empty_cache()
    log("router counters (rms replays, logit replays, gemma exact replays, exact ties):", zz.stats())

    head_leg, head_S = ("gemma", args.tokens) if "gemma" in res and args.tokens in res["gemma"] \
        else (next(iter(res)), next(iter(next(iter(res.values())))))
    r = res[head_leg][head_S]
    c = CONFIGS[head_leg]
    line = {
        "metric": f"MoE-layer tokens/s at S={head_S} (Gemma-4 q4_0, Zipf-skewed routing)"
                  if head_leg == "gemma" else f"MoE-layer tokens/s at S={head_S} ({head_leg})",
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": r["steps"],
        "warmup": args.warmup,
        "ms_per_step": r["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x q4_0 (int32 block dots, f32 scales)",
        "data": "synthetic: N(0,0.02) weights quantised to q4_0 on the device, N(0,1) inputs, "
                "seeded Zipf(1.1) router offsets",
        "config": {"workload": f"{head_leg} MoE layer d={c['D']} E={c['E']} top-{c['K']} MI={c['MI']} "
                               f"fmts {c['fmts']}, S={head_S}, {args.layers if head_leg == 'gemma' else args.cfg_layers} "
                               f"layers rotated",
                   "tokens_per_step": head_S, "mean_union_experts": r["mean_union_experts"]},
        "roofline": r["roofline"],
        "layer_roofline": r["layer_roofline"],
        "mfma": r["mfma"],
        "kernels_us": r["kernels_us"],
    }
    if "gemma" in res and 1 in res["gemma"]:
        d1 = res["gemma"][1]
        line["decode"] = dict(metric="MoE-layer tokens/s at S=1", value=d1["tokens_per_s"], unit="tokens/s",
                              us_per_step=d1["us_per_step"], kernels_us=d1["kernels_us"],
                              roofline=d1["roofline"], layer_hbm_GBs=d1["layer_roofline"]["achieved"],
                              layer_hbm_frac=d1["layer_roofline"]["frac"])
    for leg in ("lfm", "maple"):
        if leg in res:
            line[leg] = {f"S{S}": v for S, v in res[leg].items()}
            line[leg]["workload"] = (f"{leg} MoE layer d={CONFIGS[leg]['D']} E={CONFIGS[leg]['E']} "
                                     f"top-{CONFIGS[leg]['K']} MI={CONFIGS[leg]['MI']} fmts {CONFIGS[leg]['fmts']}, "
                                     f"{args.cfg_layers} layers rotated")
    if not args.no_stack and layers is not None:
        log("building and timing the gemma stack (config 5) ...")
        line["stack"] = stack_bench(zz, torch, layers, args.seed, args.tokens, args.stack_steps)
        log("stack:", json.dumps(line["stack"]))
    if not args.no_cpu and host is not None:
        log("timing the CPU reference path ...")
        line["cpu_baseline"] = cpu_baseline(zz, torch, host, args.seed, min(args.cpu_layers, len(host)))
        log("cpu:", json.dumps(line["cpu_baseline"]))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
