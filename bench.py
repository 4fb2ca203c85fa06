"""Benchmark of the quantize / block-scaled GEMM / RoPE hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,c3,c4,c5] [--no-cpu]

Workloads are BASELINE.json's five configs, on seeded synthetic inputs:
  c1  quantize_per_tensor_fp8 + dequantize_per_tensor_fp8, bf16 [4096, 3072]
  c2  apply_rope (q, k) and apply_rope1 (q), bf16 [1, 24, 4608, 128], Flux freqs
  c3  quantize_mxfp8, bf16 [4608, 3072] with per-row log-normal magnitudes   <- `value`
      (+ dequantize_mxfp8 of the result, bf16 out)
  c4  scaled_mm_mxfp8, [4608, 3072] x [12288, 3072] -> bf16
  c5  quantize_nvfp4 [8192, 5120] (+ dequantize_nvfp4 of the result)
      + scaled_mm_nvfp4 [8192, 5120] x [13824, 5120]

Timing: W untimed warmup steps, then K steps captured in one HIP graph and replayed
between HIP events on the launch stream (torch's current stream, where the ops
launch), so Python dispatch overhead is excluded and back-to-back kernel time is
what is measured.  Inputs/outputs rotate over buffer sets totalling > 512 MB so the
256 MB Infinity Cache cannot hold the working set.  Graph replays are checked
against the eager call's output before timing.

Each op line reports algorithmic bytes (or FLOPs) per call / measured time, and its
fraction of the MI355X peak (HBM 8 TB/s; dense FP8 MFMA 5.0 PF; BF16 2.5 PF).  The
CPU baseline times the CPU oracle (a restatement of the reference eager backend) on
a bounded sample on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parent
for p in (REPO / "comfy-kitchen_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
FP4_PEAK_TFLOPS = 10100.0
ROTATE_BYTES = 512 << 20
METRIC = "quantize GB/s (% HBM peak); scaled_mm_mxfp8 TFLOPS (% MFMA peak), 1 GPU"


# ------------------------------------------------------------------ workloads
def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def make_c1(device="cpu"):
    """bf16 [4096, 3072], N(0,1)*0.5 with 0.1% outliers x20; scale = amax/448 (fp32)."""
    g = gen(0)
    x = torch.randn(4096, 3072, generator=g) * 0.5
    n = x.numel()
    idx = torch.randperm(n, generator=g)[: n // 1000]
    x.view(-1)[idx] *= 20
    x = x.bfloat16()
    scale = (x.abs().amax().float() / 448.0).reshape(1)
    return x.to(device), scale.to(device)


def flux_freqs(h=72, w=64, axes=(16, 56, 56), theta=10000.0) -> torch.Tensor:
    """Flux EmbedND rotation matrices for ids (0, i, j), i < h, j < w: [1, 1, h*w, 64, 2, 2] fp32."""
    ii, jj = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
    ids = torch.stack([torch.zeros_like(ii), ii, jj], dim=-1).reshape(-1, 3).double()
    mats = []
    for a, d in enumerate(axes):
        omega = 1.0 / theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
        phi = ids[:, a:a + 1] * omega[None, :]
        m = torch.stack([torch.cos(phi), -torch.sin(phi), torch.sin(phi), torch.cos(phi)], dim=-1)
        mats.append(m.reshape(-1, d // 2, 2, 2))
    return torch.cat(mats, dim=1).float().reshape(1, 1, h * w, sum(axes) // 2, 2, 2)


def make_c2(device="cpu"):
    g = gen(1)
    q = torch.randn(1, 24, 4608, 128, generator=g).bfloat16()
    k = torch.randn(1, 24, 4608, 128, generator=g).bfloat16()
    return q.to(device), k.to(device), flux_freqs().to(device)


def make_c3(device="cpu"):
    g = gen(2)
    x = torch.randn(4608, 3072, generator=g) * torch.exp(torch.randn(4608, 1, generator=g))
    return x.bfloat16().to(device)


def make_c4_weight(device="cpu"):
    return (torch.randn(12288, 3072, generator=gen(3)) * 0.02).bfloat16().to(device)


def make_c5(device="cpu"):
    a = torch.randn(8192, 5120, generator=gen(4)).bfloat16()
    w = (torch.randn(13824, 5120, generator=gen(5)) * 0.02).bfloat16()
    ga = (a.abs().amax().float() / 2688.0).reshape(1)
    gw = (w.abs().amax().float() / 2688.0).reshape(1)
    return a.to(device), w.to(device), ga.to(device), gw.to(device)


# Algorithmic bytes / FLOPs per call (inputs read once + outputs written once).
BYTES = {
    "quantize_per_tensor_fp8": 4096 * 3072 * 3 + 4,
    "dequantize_per_tensor_fp8": 4096 * 3072 * 3 + 4,
    "apply_rope": 4 * 24 * 4608 * 128 * 2 + 4608 * 64 * 4 * 4,
    "apply_rope1": 2 * 24 * 4608 * 128 * 2 + 4608 * 64 * 4 * 4,
    "quantize_mxfp8": 4608 * 3072 * 3 + 4608 * 96,
    "dequantize_mxfp8": 4608 * 3072 * 3 + 4608 * 96,
    "quantize_nvfp4": 8192 * 5120 * 2 + 8192 * 2560 + 8192 * 320 + 4,
    "dequantize_nvfp4": 8192 * 5120 * 2 + 8192 * 2560 + 8192 * 320 + 4,
}
FLOPS = {
    "scaled_mm_mxfp8": 2 * 4608 * 12288 * 3072,
    "scaled_mm_nvfp4": 2 * 8192 * 13824 * 5120,
}
# (bytes read, bytes written) per call of each streaming op: the copy floor moves the same.
READ_WRITE = {
    "quantize_per_tensor_fp8": (4096 * 3072 * 2 + 4, 4096 * 3072),
    "dequantize_per_tensor_fp8": (4096 * 3072 + 4, 4096 * 3072 * 2),
    "apply_rope": (2 * 24 * 4608 * 128 * 2 + 4608 * 64 * 4 * 4, 2 * 24 * 4608 * 128 * 2),
    "apply_rope1": (24 * 4608 * 128 * 2 + 4608 * 64 * 4 * 4, 24 * 4608 * 128 * 2),
    "quantize_mxfp8": (4608 * 3072 * 2, 4608 * 3072 + 4608 * 96),
    "dequantize_mxfp8": (4608 * 3072 + 4608 * 96, 4608 * 3072 * 2),
    "quantize_nvfp4": (8192 * 5120 * 2 + 4, 8192 * 2560 + 8192 * 320),
    "dequantize_nvfp4": (8192 * 2560 + 8192 * 320 + 4, 8192 * 5120 * 2),
}
assert all(r + w == BYTES[k] for k, (r, w) in READ_WRITE.items())


# ------------------------------------------------------------------ timing
def _sets_for(bytes_per_set: int) -> int:
    return max(2, math.ceil(ROTATE_BYTES / max(bytes_per_set, 1)))


SETTLE_S = 0.3


REPLAY_ROUNDS = 5


def capture_graph(make_call, n_sets: int, steps: int, warmup: int, check=None):
    """(graph, stream) of `steps` calls, `make_call(i)` returning a zero-arg launcher for
    buffer set i; the first replay is checked with `check(outputs)`.

    Before the W warmup calls the op runs for SETTLE_S seconds so the GPU leaves its
    idle clock state (an MI355X ramps its clock over tens of milliseconds; timing a
    freshly woken GPU understates kernels by up to ~15%)."""
    calls = [make_call(i) for i in range(n_sets)]
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        for c in calls:
            c()
        torch.cuda.synchronize()
    for i in range(warmup):
        calls[i % n_sets]()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        calls[0]()  # warm the capture stream's allocator pool
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            # Only the last n_sets outputs stay referenced, so the graph's pool hands the
            # older output buffers to later calls, as the caching allocator does for eager
            # calls: outputs rotate over n_sets + 1 buffers like the inputs (and like the
            # copy floor's destinations) instead of K fresh ones.
            outs = []
            for i in range(steps):
                outs.append(calls[i % n_sets]())
                if len(outs) > n_sets:
                    outs.pop(0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    if check is not None:
        check(outs)
    return graph, stream


def time_replays(graphs, steps: int, rounds: int = REPLAY_ROUNDS) -> list[float]:
    """ms per call of each captured graph: after SETTLE_S of replays of all of them, `rounds`
    timed replays of each, in alternating order (ABBA), each one replay of K calls between
    HIP events on the graph's stream; the median replay is reported.  Graphs compared with
    each other (an op and its copy floor) thus run under the same clock and memory state."""
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        for g, _ in graphs:
            g.replay()
        torch.cuda.synchronize()
    res = [[] for _ in graphs]
    for r in range(rounds):
        order = range(len(graphs)) if r % 2 == 0 else reversed(range(len(graphs)))
        for j in order:
            graph, stream = graphs[j]
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                start.record(stream)
                graph.replay()
                end.record(stream)
            torch.cuda.synchronize()
            res[j].append(start.elapsed_time(end) / steps)
    return [sorted(x)[len(x) // 2] for x in res]


def time_graph(make_call, n_sets: int, steps: int, warmup: int, check=None) -> float:
    """Median ms per call of a graph of `steps` calls (capture_graph, time_replays)."""
    return time_replays([capture_graph(make_call, n_sets, steps, warmup, check)], steps)[0]


def time_cpu(fn, min_reps=3, budget_s=3.0) -> tuple[float, int]:
    """Median seconds per call of fn() on the CPU: repeated for budget_s (at least min_reps
    calls) after one warmup call."""
    fn()
    ts = []
    t_all = time.perf_counter()
    while len(ts) < min_reps or time.perf_counter() - t_all < budget_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], len(ts)


_bench_lib = None


def bench_lib():
    """comfy-kitchen_amd/benchlib/libckh_bench.so: kernels timed only for comparison."""
    global _bench_lib
    if _bench_lib is None:
        import ctypes

        lib = ctypes.CDLL(str(REPO / "comfy-kitchen_amd" / "benchlib" / "libckh_bench.so"))
        lib.ckh_bench_copy_floor.restype = ctypes.c_int
        lib.ckh_bench_copy_floor.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64,
                                             ctypes.c_uint64]
        lib.ckh_bench_mfma_loop.restype = ctypes.c_int
        lib.ckh_bench_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_uint64]
        _bench_lib = lib
    return _bench_lib


def copy_floor_calls(read_bytes: int, write_bytes: int):
    """(make_call, n_sets) of a streaming copy that reads and writes the given bytes, over
    buffer sets rotating through > 512 MB like the ops' (benchlib/copy_floor.hip)."""
    lib = bench_lib()
    dev = torch.device("cuda", 0)
    nset = _sets_for(read_bytes + write_bytes)
    srcs = [torch.randint(0, 255, (read_bytes,), dtype=torch.uint8, device=dev) for _ in range(nset)]
    dsts = [torch.empty(write_bytes, dtype=torch.uint8, device=dev) for _ in range(nset)]

    def make(i):
        def call():
            st = torch.cuda.current_stream().cuda_stream
            if lib.ckh_bench_copy_floor(srcs[i].data_ptr(), read_bytes, dsts[i].data_ptr(), write_bytes, st):
                raise RuntimeError("copy floor launch failed")
            return dsts[i]
        return call

    return make, nset


def vendor_copy_calls(nbytes: int):
    """(make_call, n_sets) of torch's own device copy (Tensor.copy_ on uint8 tensors) of
    nbytes, reading and writing nbytes each, over buffer sets rotating through > 512 MB."""
    dev = torch.device("cuda", 0)
    nset = _sets_for(2 * nbytes)
    srcs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev) for _ in range(nset)]
    dsts = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(nset)]

    def make(i):
        def call():
            return dsts[i].copy_(srcs[i])
        return call

    return make, nset


def time_with_floor(name: str, make_call, n_sets: int, steps: int, warmup: int, check=None) -> tuple[float, dict]:
    """(ms per call of the op, {"ours": ms of the copy floor for its bytes, "vendor": ms of
    torch's device copy moving the same total bytes}): the three graphs captured, then timed
    in alternating rounds (time_replays)."""
    g_op = capture_graph(make_call, n_sets, steps, warmup, check)
    rd, wr = READ_WRITE[name]
    fmake, fn = copy_floor_calls(rd, wr)
    g_floor = capture_graph(fmake, fn, steps, warmup)
    vmake, vn = vendor_copy_calls((rd + wr) // 2)
    g_vendor = capture_graph(vmake, vn, steps, warmup)
    ms, floor, vendor = time_replays([g_op, g_floor, g_vendor], steps)
    return ms, {"ours": floor, "vendor": vendor}


def record_floor(res: dict, name: str, floor: dict, log) -> None:
    res[name]["copy_floor_ms"] = floor["ours"]
    res[name]["of_copy_floor"] = round(floor["ours"] / res[name]["ms"], 4)
    res[name]["vendor_copy_ms"] = floor["vendor"]
    res[name]["of_vendor_copy"] = round(floor["vendor"] / res[name]["ms"], 4)
    log(f"   copy floor for {name}'s bytes: {floor['ours'] * 1e3:.2f} us ({res[name]['of_copy_floor'] * 100:.1f}% of "
        f"it); torch copy_ of the same bytes: {floor['vendor'] * 1e3:.2f} us ({res[name]['of_vendor_copy'] * 100:.1f}%)")


def roofline_bytes(nbytes, ms, traffic=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}


def roofline_flops(flops, ms, peak, traffic=None):
    tf = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(tf / peak, 4), "traffic": traffic}


def load_traffic() -> dict:
    """Bytes per launch that missed L2, measured with rocprofv3 --pmc (TCC FETCH_SIZE + WRITE_SIZE), if
    recorded: HBM traffic plus Infinity-Cache (MALL) hits, i.e. an upper bound on HBM bytes."""
    p = REPO / "profiles" / "traffic.json"
    if p.exists():
        try:
            per = json.loads(p.read_text()).get("bytes_per_launch", {})
            return {k: v.get("total") for k, v in per.items()}
        except (ValueError, OSError, AttributeError):
            return {}
    return {}


# ------------------------------------------------------------------ GEMMs
# Flux / Wan-14B linear shapes (M, N, K) the reference's model patchers quantize
# (samples/mxfp8_model_patcher.py:78-117 patches every nn.Linear): Flux double-block qkv,
# projection, MLP up / down at 4608 image tokens; the modulation linears at batch 1 and 16;
# Wan-14B attention and FFN at 8192 tokens.
LINEAR_SHAPES = [
    ("flux_qkv", 4608, 9216, 3072), ("flux_proj", 4608, 3072, 3072), ("flux_mlp_up", 4608, 12288, 3072),
    ("flux_mlp_down", 4608, 3072, 12288), ("flux_mod_m1", 1, 18432, 3072), ("flux_mod_m16", 16, 18432, 3072),
    ("wan_attn", 8192, 5120, 5120), ("wan_ffn_up", 8192, 13824, 5120), ("wan_ffn_down", 8192, 5120, 13824),
    # short activations (e.g. a text prompt's tokens): small tile grids, split-K or half tiles
    ("m256_flux_mod", 256, 18432, 3072), ("m256_wan_ffn_up", 256, 13824, 5120), ("m256_wan_ffn_down", 256, 5120, 13824),
    ("m64_flux_mod", 64, 18432, 3072),
]
# NVFP4 linears (no vendor NVFP4 GEMM on this stack): skinny, split-K and full tile grids
NV_LINEAR_SHAPES = [
    ("wan_ffn_up_m1", 1, 13824, 5120), ("wan_ffn_up_m16", 16, 13824, 5120), ("wan_ffn_up_m64", 64, 13824, 5120),
    ("wan_ffn_up_m256", 256, 13824, 5120), ("wan_ffn_down_m256", 256, 5120, 13824), ("flux_mod_m1", 1, 18432, 3072),
    ("wan_ffn_down_m16", 16, 5120, 13824), ("wan_ffn_down_m64", 64, 5120, 13824),
]


def gemm_operands(m: int, n: int, k: int, seed: int, dev):
    """MXFP8 operands of a linear: activation N(0, 1), weight N(0, 0.02), both bf16 quantized
    by ck.quantize_mxfp8 (seeded, generated on the device)."""
    import comfy_kitchen as ck

    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(m, k, device=dev, generator=g).bfloat16()
    w = (torch.randn(n, k, device=dev, generator=g) * 0.02).bfloat16()
    qa, sa = ck.quantize_mxfp8(x)
    qw, sw = ck.quantize_mxfp8(w)
    return qa, sa, qw, sw


def time_gemm_variants(qa, sa, qw, sw, steps: int, warmup: int, vendor: bool = True) -> dict:
    """ms per call of ck.scaled_mm_mxfp8 ("mx"), ck.scaled_mm_fp8 with unit tensor scales
    ("fp8"), and the vendor GEMMs the reference calls on a GPU: torch._scaled_mm tensor-wise
    ("vendor_fp8", TensorCoreFP8Layout's F.scaled_mm path) and torch's F.scaled_mm with 1 x 32
    E8M0 scales ("vendor_mx", eager scaled_mm_mxfp8), each a HIP graph over rotating operand
    sets.  The vendor MX GEMM reads row-major (unswizzled) scales: with the reference's
    SWIZZLE_32_4_4 argument on these swizzled scales, torch on ROCm returns wrong results,
    whose rel-L2 against ours is recorded as "vendor_mx_reference_call_rel_l2"."""
    import torch.nn.functional as F

    import comfy_kitchen as ck

    m, k = qa.shape
    n = qw.shape[0]
    nset = _sets_for(qa.numel() + qw.numel())
    sets = [(qa.clone(), qw.clone(), sa.clone(), sw.clone()) for _ in range(nset)]
    one = torch.ones(1, device=qa.device)
    k_steps = max(steps // 2, 10)
    out = {}
    ref = ck.scaled_mm_mxfp8(qa, qw, sa, sw)

    def same(outs):
        for o in outs:
            if not torch.equal(o, ref):
                sys.exit("graph replay mismatch in a GEMM")

    cands = [("mx", lambda i: (lambda: ck.scaled_mm_mxfp8(*sets[i])), same),
             ("fp8", lambda i: (lambda: ck.scaled_mm_fp8(sets[i][0], sets[i][1], one, one)), None)]
    if vendor:
        one0 = one.reshape(())
        cands.append(("vendor_fp8", lambda i: (lambda: torch._scaled_mm(sets[i][0], sets[i][1].t(), one0, one0,
                                                                        out_dtype=torch.bfloat16)), None))
        try:
            sa_p = ck.from_blocked(sa.view(torch.uint8), m, k // 32).contiguous().view(torch.float8_e8m0fnu)
            sw_p = ck.from_blocked(sw.view(torch.uint8), n, k // 32).contiguous().view(torch.float8_e8m0fnu)

            def vmx(a, b, x, y, swz):
                return F.scaled_mm(a, b.t(), scale_a=x, scale_recipe_a=F.ScalingType.BlockWise1x32, scale_b=y,
                                   scale_recipe_b=F.ScalingType.BlockWise1x32, swizzle_a=swz, swizzle_b=swz,
                                   output_dtype=torch.bfloat16)
            rel = lambda o: round(float((o.float() - ref.float()).norm() / ref.float().norm()), 5)  # noqa: E731
            out["vendor_mx_rel_l2"] = rel(vmx(qa, qw, sa_p, sw_p, F.SwizzleType.NO_SWIZZLE))
            out["vendor_mx_reference_call_rel_l2"] = rel(vmx(qa, qw, sa, sw, F.SwizzleType.SWIZZLE_32_4_4))
            cands.append(("vendor_mx", lambda i: (lambda: vmx(sets[i][0], sets[i][1], sa_p, sw_p,
                                                              F.SwizzleType.NO_SWIZZLE)), None))
        except (RuntimeError, ValueError) as e:
            out["vendor_mx_error"] = str(e)[:200]
    graphs, names = [], []
    for name, make, chk in cands:
        try:
            graphs.append(capture_graph(make, nset, k_steps, warmup, chk))
            names.append(name)
        except (RuntimeError, ValueError) as e:
            out[f"{name}_error"] = str(e)[:200]
    for name, ms in zip(names, time_replays(graphs, k_steps)):
        out[f"{name}_ms"] = ms
    del sets, graphs
    return out


def run_linear_shapes(steps: int, warmup: int, log) -> dict:
    """ops.linear_shapes: each LINEAR_SHAPES entry's GEMM times (time_gemm_variants), TFLOPS
    and fraction of the dense FP8 peak; for M <= 256 also the weight bytes (codes + scales)
    per second and their fraction of HBM peak."""
    dev = torch.device("cuda", 0)
    res = {}
    for i, (name, m, n, k) in enumerate(LINEAR_SHAPES):
        qa, sa, qw, sw = gemm_operands(m, n, k, 100 + i, dev)
        t = time_gemm_variants(qa, sa, qw, sw, steps, warmup)
        flops = 2 * m * n * k
        e = {"M": m, "N": n, "K": k}
        for key in ("mx", "fp8", "vendor_fp8", "vendor_mx"):
            if f"{key}_ms" in t:
                ms = t[f"{key}_ms"]
                e[key] = {"ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                          "frac_fp8_peak": round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4)}
                if m <= 256:
                    wb = qw.numel() + sw.numel()
                    gbs = wb / (ms * 1e-3) / 1e9
                    e[key].update({"weight_gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        e.update({k2: v for k2, v in t.items() if not k2.endswith("_ms")})
        res[name] = e
        log(f"linear {name} [{m}, {n}, {k}]: " + ", ".join(
            f"{key} {e[key]['ms'] * 1e3:.1f} us" for key in ("mx", "fp8", "vendor_fp8", "vendor_mx") if key in e))
        del qa, sa, qw, sw
    return res


def run_nv_linear_shapes(steps: int, warmup: int, log) -> dict:
    """ops.nv_linear_shapes: ck.scaled_mm_nvfp4 on each NV_LINEAR_SHAPES entry (bf16 operands
    N(0, 1) and N(0, 0.02) quantized by ck.quantize_nvfp4 with amax/2688 global scales), graph-
    timed over rotating weight sets: TFLOPS against the dense f16 peak the kernel computes at,
    and for M <= 256 the weight bytes (codes + scales) per second against HBM peak."""
    import comfy_kitchen as ck

    dev = torch.device("cuda", 0)
    res = {}
    for i, (name, m, n, k) in enumerate(NV_LINEAR_SHAPES):
        g = torch.Generator(device=dev).manual_seed(200 + i)
        x = torch.randn(m, k, device=dev, generator=g).bfloat16()
        w = (torch.randn(n, k, device=dev, generator=g) * 0.02).bfloat16()
        gx, gw = ck.amax_scale(x, 2688.0), ck.amax_scale(w, 2688.0)
        qa, sa = ck.quantize_nvfp4(x, gx)
        qw, sw = ck.quantize_nvfp4(w, gw)
        ref = ck.scaled_mm_nvfp4(qa, qw, gx, gw, sa, sw)
        nset = _sets_for(qa.numel() + qw.numel())
        ws = [(qw.clone(), sw.clone()) for _ in range(nset)]
        ms = time_graph(lambda i_: (lambda: ck.scaled_mm_nvfp4(qa, ws[i_][0], gx, gw, sa, ws[i_][1])), nset,
                        max(steps // 2, 10), warmup,
                        check=lambda outs: [torch.equal(o, ref) or sys.exit("graph mismatch nv linear") for o in outs])
        flops = 2 * m * n * k
        wb = qw.numel() + sw.numel()
        e = {"M": m, "N": n, "K": k, "ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
             "frac_f16_peak": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}
        if m <= 256:
            gbs = wb / (ms * 1e-3) / 1e9
            e.update({"weight_gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        res[name] = e
        log(f"nv linear {name} [{m}, {n}, {k}]: {ms * 1e3:.1f} us")
        del ws, x, w, qa, sa, qw, sw
    return res


def run_copy_sweep(log) -> dict:
    """The two copies (benchlib/copy_floor.hip and torch's Tensor.copy_), each moving S bytes
    (S/2 read + S/2 written) for S from 32 MB to 1 GB, graph-timed over rotating buffers, and
    a least-squares fit t = fixed + S / rate per copy: the fixed per-call cost and the
    asymptotic rate that bound a streaming kernel of a given size."""
    sizes = [32 << 20, 64 << 20, 128 << 20, 256 << 20, 512 << 20, 1024 << 20]
    out = {"bytes_moved": sizes, "ours_us": [], "vendor_us": []}
    for sz in sizes:
        fmake, fn = copy_floor_calls(sz // 2, sz // 2)
        vmake, vn = vendor_copy_calls(sz // 2)
        steps = 20
        g1 = capture_graph(fmake, fn, steps, 3)
        g2 = capture_graph(vmake, vn, steps, 3)
        a, b = time_replays([g1, g2], steps)
        out["ours_us"].append(round(a * 1e3, 2))
        out["vendor_us"].append(round(b * 1e3, 2))
        del g1, g2
    for key in ("ours", "vendor"):
        ts = out[f"{key}_us"]
        n = len(sizes)
        mx_, my = sum(sizes) / n, sum(ts) / n
        slope = sum((x - mx_) * (y - my) for x, y in zip(sizes, ts)) / sum((x - mx_) ** 2 for x in sizes)
        out[f"{key}_fit"] = {"fixed_us": round(my - slope * mx_, 2), "rate_gbs": round(1e-3 / slope, 1)}
    log(f"copy sweep: ours {out['ours_fit']}, torch copy_ {out['vendor_fit']}")
    return out


# ------------------------------------------------------------------ runs
def run_gpu(configs, steps, warmup, log):
    import comfy_kitchen as ck

    # Each timed graph's replay is checked, bit for bit, against the same op called eagerly.
    dev = torch.device("cuda", 0)
    res = {}
    traffic = load_traffic()

    def same(a, b):
        return torch.equal(a.view(torch.uint8) if a.element_size() == 1 else a, b.view(torch.uint8) if b.element_size() == 1 else b)

    if "c1" in configs:
        x, scale = make_c1(dev)
        nset = _sets_for(BYTES["quantize_per_tensor_fp8"])
        xs = [x.clone() for _ in range(nset)]
        ref_q = ck.quantize_per_tensor_fp8(x, scale)
        ms, floor = time_with_floor(
            "quantize_per_tensor_fp8", lambda i: (lambda: ck.quantize_per_tensor_fp8(xs[i], scale)), nset, steps,
            warmup, check=lambda outs: [same(o, ref_q) or sys.exit("graph replay mismatch c1 q") for o in outs])
        res["quantize_per_tensor_fp8"] = {"ms": ms, **roofline_bytes(BYTES["quantize_per_tensor_fp8"], ms,
                                                                      traffic.get("quantize_per_tensor_fp8"))}
        log(f"c1 quantize_per_tensor_fp8: {ms * 1e3:.2f} us")
        record_floor(res, "quantize_per_tensor_fp8", floor, log)
        qs = [ref_q.clone() for _ in range(nset)]
        ref_dq = ck.dequantize_per_tensor_fp8(ref_q, scale)
        ms, floor = time_with_floor(
            "dequantize_per_tensor_fp8", lambda i: (lambda: ck.dequantize_per_tensor_fp8(qs[i], scale)), nset, steps,
            warmup, check=lambda outs: [same(o, ref_dq) or sys.exit("graph replay mismatch c1 dq") for o in outs])
        res["dequantize_per_tensor_fp8"] = {"ms": ms, **roofline_bytes(BYTES["dequantize_per_tensor_fp8"], ms,
                                                                        traffic.get("dequantize_per_tensor_fp8"))}
        log(f"c1 dequantize_per_tensor_fp8: {ms * 1e3:.2f} us")
        record_floor(res, "dequantize_per_tensor_fp8", floor, log)
        del xs, qs

    if "c2" in configs:
        q, k, f = make_c2(dev)
        nset = _sets_for(BYTES["apply_rope"])
        qs = [q.clone() for _ in range(nset)]
        ks = [k.clone() for _ in range(nset)]
        rq, rk = ck.apply_rope(q, k, f)
        ms, floor = time_with_floor(
            "apply_rope", lambda i: (lambda: ck.apply_rope(qs[i], ks[i], f)), nset, steps, warmup,
            check=lambda outs: [(same(a, rq) and same(b, rk)) or sys.exit("graph mismatch c2") for a, b in outs])
        res["apply_rope"] = {"ms": ms, **roofline_bytes(BYTES["apply_rope"], ms, traffic.get("apply_rope"))}
        log(f"c2 apply_rope: {ms * 1e3:.2f} us")
        record_floor(res, "apply_rope", floor, log)
        rq1 = ck.apply_rope1(q, f)
        ms, floor = time_with_floor(
            "apply_rope1", lambda i: (lambda: ck.apply_rope1(qs[i], f)), nset, steps, warmup,
            check=lambda outs: [same(o, rq1) or sys.exit("graph mismatch c2 rope1") for o in outs])
        res["apply_rope1"] = {"ms": ms, **roofline_bytes(BYTES["apply_rope1"], ms, traffic.get("apply_rope1"))}
        log(f"c2 apply_rope1: {ms * 1e3:.2f} us")
        record_floor(res, "apply_rope1", floor, log)
        del qs, ks

    if "c3" in configs or "c4" in configs:
        x = make_c3(dev)
        qa, sa = ck.quantize_mxfp8(x)
        if "c3" in configs:
            nset = _sets_for(BYTES["quantize_mxfp8"])
            xs = [x.clone() for _ in range(nset)]
            ms, floor = time_with_floor(
                "quantize_mxfp8", lambda i: (lambda: ck.quantize_mxfp8(xs[i])), nset, steps, warmup,
                check=lambda outs: [(same(a, qa) and same(b, sa)) or sys.exit("graph mismatch c3") for a, b in outs])
            res["quantize_mxfp8"] = {"ms": ms, **roofline_bytes(BYTES["quantize_mxfp8"], ms,
                                                                 traffic.get("quantize_mxfp8"))}
            log(f"c3 quantize_mxfp8: {ms * 1e3:.2f} us")
            record_floor(res, "quantize_mxfp8", floor, log)
            del xs
            # the layouts' dequantize of the same tensor (bf16 out)
            want = ck.dequantize_mxfp8(qa, sa)
            nset = _sets_for(BYTES["dequantize_mxfp8"])
            qs_ = [(qa.clone(), sa.clone()) for _ in range(nset)]
            ms, floor = time_with_floor(
                "dequantize_mxfp8", lambda i: (lambda: ck.dequantize_mxfp8(*qs_[i])), nset, steps, warmup,
                check=lambda outs: [same(o, want) or sys.exit("graph mismatch c3 dequantize") for o in outs])
            res["dequantize_mxfp8"] = {"ms": ms, **roofline_bytes(BYTES["dequantize_mxfp8"], ms,
                                                                   traffic.get("dequantize_mxfp8"))}
            log(f"c3 dequantize_mxfp8: {ms * 1e3:.2f} us")
            record_floor(res, "dequantize_mxfp8", floor, log)
            del qs_, want
        if "c4" in configs:
            qw, sw = ck.quantize_mxfp8(make_c4_weight(dev))
            try:
                ref = ck.scaled_mm_mxfp8(qa, qw, sa, sw)
                nset = _sets_for(qa.numel() + qw.numel())
                ops_ = [(qa.clone(), qw.clone(), sa.clone(), sw.clone()) for _ in range(nset)]
                ms = time_graph(lambda i: (lambda: ck.scaled_mm_mxfp8(*ops_[i])), nset, max(steps // 4, 5),
                                warmup, check=lambda outs: [same(o, ref) or sys.exit("graph mismatch c4") for o in outs])
                del ops_
                res["scaled_mm_mxfp8"] = {"ms": ms, **roofline_flops(FLOPS["scaled_mm_mxfp8"], ms, FP8_PEAK_TFLOPS,
                                                                      traffic.get("scaled_mm_mxfp8"))}
                log(f"c4 scaled_mm_mxfp8: {ms * 1e3:.1f} us")
                # the same shape through ck.scaled_mm_fp8 and the vendor GEMMs, in one set of
                # alternating rounds
                t = time_gemm_variants(qa, sa, qw, sw, steps, warmup)
                for key, name in (("mx", "scaled_mm_mxfp8_same_run"), ("fp8", "scaled_mm_fp8"),
                                  ("vendor_fp8", "scaled_mm_fp8_vendor"), ("vendor_mx", "scaled_mm_mxfp8_vendor")):
                    if f"{key}_ms" in t:
                        res[name] = {"ms": t[f"{key}_ms"], **roofline_flops(FLOPS["scaled_mm_mxfp8"], t[f"{key}_ms"],
                                                                         FP8_PEAK_TFLOPS)}
                res["scaled_mm_mxfp8_vendor"] = {**res.get("scaled_mm_mxfp8_vendor", {}),
                                                 **{k2: v for k2, v in t.items() if k2.startswith("vendor_mx_")},
                                                 "what": "torch F.scaled_mm, BlockWise1x32 E8M0, row-major scales"}
                res["scaled_mm_fp8_vendor"] = {**res.get("scaled_mm_fp8_vendor", {}),
                                               "what": "torch._scaled_mm tensor-wise FP8 (C4 codes, unit scales)"}
                log("c4 same run: " + ", ".join(f"{k2} {v * 1e3:.1f} us" for k2, v in t.items() if k2.endswith("_ms")))
            except RuntimeError as e:
                res["scaled_mm_mxfp8"] = {"error": str(e)}
                log(f"c4 scaled_mm_mxfp8 unavailable: {e}")

    if "c5" in configs:
        a, w, ga, gw = make_c5(dev)
        qa, sa = ck.quantize_nvfp4(a, ga)
        nset = _sets_for(BYTES["quantize_nvfp4"])
        as_ = [a.clone() for _ in range(nset)]
        ms, floor = time_with_floor(
            "quantize_nvfp4", lambda i: (lambda: ck.quantize_nvfp4(as_[i], ga)), nset, steps, warmup,
            check=lambda outs: [(same(x_, qa) and same(y_, sa)) or sys.exit("graph mismatch c5") for x_, y_ in outs])
        res["quantize_nvfp4"] = {"ms": ms, **roofline_bytes(BYTES["quantize_nvfp4"], ms, traffic.get("quantize_nvfp4"))}
        log(f"c5 quantize_nvfp4: {ms * 1e3:.2f} us")
        record_floor(res, "quantize_nvfp4", floor, log)
        # dynamic scale (the layouts' scale=None): the fused call against amax_scale + quantize
        g_dyn = ck.amax_scale(a, 2688.0)
        q_dyn, s_dyn = ck.quantize_nvfp4(a, g_dyn)

        def check_dyn(outs):
            for o in outs:
                q_, s_, g_ = o if len(o) == 3 else (*o, None)
                if not (same(q_, q_dyn) and same(s_, s_dyn)) or (g_ is not None and not torch.equal(g_, g_dyn)):
                    sys.exit("graph mismatch c5 dynamic")

        ms_fused = time_graph(lambda i: (lambda: ck.quantize_nvfp4_dynamic(as_[i], 2688.0)), nset, steps, warmup,
                              check=check_dyn)
        ms_two = time_graph(lambda i: (lambda: ck.quantize_nvfp4(as_[i], ck.amax_scale(as_[i], 2688.0))), nset,
                            steps, warmup, check=check_dyn)
        res["quantize_nvfp4_dynamic"] = {
            "ms": ms_fused, **roofline_bytes(BYTES["quantize_nvfp4"], ms_fused),
            "two_call_ms": ms_two, "note": "amax(|x|)/2688 + quantize_nvfp4 in two launches (x re-read from the "
                                           "infinity cache) vs amax_scale (2 launches) + quantize_nvfp4"}
        log(f"c5 quantize_nvfp4_dynamic: {ms_fused * 1e3:.2f} us fused vs {ms_two * 1e3:.2f} us amax_scale + quantize")
        del as_
        want = ck.dequantize_nvfp4(qa, ga, sa)
        nset = _sets_for(BYTES["dequantize_nvfp4"])
        qs_ = [(qa.clone(), sa.clone()) for _ in range(nset)]
        ms, floor = time_with_floor(
            "dequantize_nvfp4", lambda i: (lambda: ck.dequantize_nvfp4(qs_[i][0], ga, qs_[i][1])), nset, steps,
            warmup, check=lambda outs: [same(o, want) or sys.exit("graph mismatch c5 dequantize") for o in outs])
        res["dequantize_nvfp4"] = {"ms": ms, **roofline_bytes(BYTES["dequantize_nvfp4"], ms,
                                                               traffic.get("dequantize_nvfp4"))}
        log(f"c5 dequantize_nvfp4: {ms * 1e3:.2f} us")
        record_floor(res, "dequantize_nvfp4", floor, log)
        del qs_, want
        qw, sw = ck.quantize_nvfp4(w, gw)
        try:
            ref = ck.scaled_mm_nvfp4(qa, qw, ga, gw, sa, sw)
            nset = _sets_for(qa.numel() + qw.numel())
            ops_ = [(qa.clone(), qw.clone(), sa.clone(), sw.clone()) for _ in range(nset)]
            ms = time_graph(lambda i: (lambda: ck.scaled_mm_nvfp4(ops_[i][0], ops_[i][1], ga, gw, ops_[i][2], ops_[i][3])),
                            nset, max(steps // 4, 5), warmup,
                            check=lambda outs: [same(o, ref) or sys.exit("graph mismatch c5 mm") for o in outs])
            del ops_
            r = roofline_flops(FLOPS["scaled_mm_nvfp4"], ms, BF16_PEAK_TFLOPS, traffic.get("scaled_mm_nvfp4"))
            r["frac_of_fp4_peak"] = round(r["achieved"] / FP4_PEAK_TFLOPS, 4)
            res["scaled_mm_nvfp4"] = {"ms": ms, **r}
            log(f"c5 scaled_mm_nvfp4: {ms * 1e3:.1f} us")
        except RuntimeError as e:
            res["scaled_mm_nvfp4"] = {"error": str(e)}
            log(f"c5 scaled_mm_nvfp4 unavailable: {e}")
    return res


def host_info() -> dict:
    """CPU model (the model-name string plus family / model / stepping, since a virtualised
    host may shorten the name), logical CPU count, torch's CPU vector capability (it sets the
    eager kernels' vector width) and torch version of this host."""
    info = {}
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                key, _, val = line.partition(":")
                key = key.strip()
                if key in ("model name", "cpu family", "model", "stepping", "vendor_id") and key not in info:
                    info[key] = val.strip()
                if not line.strip() and info:
                    break
    except OSError:
        pass
    try:
        cap = torch.backends.cpu.get_cpu_capability()
    except (AttributeError, RuntimeError):
        cap = ""
    model = info.get("model name", "")
    ident = ", ".join(f"{k} {info[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in info)
    return {"cpu_model": f"{model} ({ident})" if ident else model, "host_cpus": os.cpu_count(),
            "torch_cpu_capability": cap, "torch": torch.__version__}


def run_cpu_baseline(configs, log):
    """Time the CPU oracle (restatement of the reference eager path) on bounded samples.

    Threads: the host share of a one-GPU box, OMP_NUM_THREADS (16 there), rather than
    os.cpu_count(), which counts every CPU of a host shared by several GPU boxes; both are
    recorded with each figure."""
    from oracle import eager_ref as ref

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1))
    cores = torch.get_num_threads()
    host = host_info()
    out = {}

    def put(name, value, unit, sample):
        out[name] = {"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample, **host}
        log(f"cpu {name}: {value} {unit} ({sample})")

    def gbs(name, nbytes, fn, sample, **kw):
        s, reps = time_cpu(fn, **kw)
        put(name, round(nbytes / s / 1e9, 3), "GB/s", f"{sample}, median of {reps} runs")

    if "c3" in configs:
        x = make_c3()
        gbs("quantize_mxfp8", BYTES["quantize_mxfp8"], lambda: ref.quantize_mxfp8(x),
            "full C3 tensor [4608, 3072] bf16 (~12 s of CPU work)", budget_s=12.0)
        q, sc = ref.quantize_mxfp8(x)
        gbs("dequantize_mxfp8", BYTES["dequantize_mxfp8"], lambda: ref.dequantize_mxfp8(q, sc, torch.bfloat16),
            "full C3 codes and scales, bf16 out")
    if "c1" in configs:
        x, scale = make_c1()
        gbs("quantize_per_tensor_fp8", BYTES["quantize_per_tensor_fp8"],
            lambda: ref.quantize_per_tensor_fp8(x, scale), "full C1 tensor")
        q = ref.quantize_per_tensor_fp8(x, scale)
        gbs("dequantize_per_tensor_fp8", BYTES["dequantize_per_tensor_fp8"],
            lambda: ref.dequantize_per_tensor_fp8(q, scale, torch.bfloat16), "full C1 codes, bf16 out")
    if "c2" in configs:
        q, k, f = make_c2()
        gbs("apply_rope", BYTES["apply_rope"], lambda: ref.apply_rope(q, k, f), "full C2 q, k")
        gbs("apply_rope1", BYTES["apply_rope1"], lambda: ref.apply_rope1(q, f), "full C2 q")
    if "c5" in configs:
        a_full, w_full, _, _ = make_c5()
        a = a_full[:1024]
        ga = (a.abs().amax().float() / 2688).reshape(1)
        gbs("quantize_nvfp4", BYTES["quantize_nvfp4"] // 8, lambda: ref.quantize_nvfp4(a, ga),
            "first 1024 of 8192 rows of C5 A")
        qa, sa = ref.quantize_nvfp4(a, ga)
        gbs("dequantize_nvfp4", BYTES["dequantize_nvfp4"] // 8,
            lambda: ref.dequantize_nvfp4(qa, ga, sa, torch.bfloat16), "first 1024 of 8192 rows of C5 A, bf16 out")
        # eager scaled_mm has no CPU kernel; stand-in: dequantize both operands, fp32 matmul
        w = w_full[:1024]
        gw = (w.abs().amax().float() / 2688).reshape(1)
        qw, sw = ref.quantize_nvfp4(w, gw)
        qa2, sa2 = qa[:256].contiguous(), ref.to_blocked(ref.from_blocked(sa, 1024, 320)[:256].contiguous())
        s, reps = time_cpu(lambda: ref.scaled_mm_nvfp4_ref(qa2, qw, ga, gw, sa2, sw), min_reps=1, budget_s=5.0)
        put("scaled_mm_nvfp4", round(2 * 256 * 1024 * 5120 / s / 1e12, 4), "TFLOP/s",
            f"256 of 8192 rows of A x 1024 of 13824 rows of W: dequantize both + fp32 matmul, median of {reps}")
        del a_full, w_full
    if "c4" in configs:
        x = make_c3()[:512]
        wq, ws = ref.quantize_mxfp8(make_c4_weight())
        xq, xs = ref.quantize_mxfp8(x)
        s, reps = time_cpu(lambda: ref.scaled_mm_mxfp8_ref(xq, wq, xs, ws), min_reps=1, budget_s=5.0)
        put("scaled_mm_mxfp8", round(2 * 512 * 12288 * 3072 / s / 1e12, 4), "TFLOP/s",
            f"512 of 4608 rows of A: dequantize both + fp32 matmul, median of {reps}")
    return out


# ------------------------------------------------------------------ PMC traffic
# `--pmc-driver` makes the dispatch sequence that two rocprofv3 --pmc passes count
# (FETCH_SIZE, then WRITE_SIZE); `--summarize-pmc` turns them into L2-miss bytes per launch
# (what the L2s fetch from and write to the fabric: HBM plus Infinity-Cache hits)
# in profiles/traffic.json, which the roofline lines report as `traffic`.
PMC_CALLS = 3
PMC_CALIB_BYTES = 256 << 20
PMC_MFMA_ITERS = 4000  # 64,000 MFMAs per wave, ~2 ms
# the one-pass SQ counter set of `--summarize-counters` (at most 8 SQ counters per pass)
SQ_COUNTERS = ("SQ_WAVES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS "
               "SQ_LDS_BANK_CONFLICT SQ_LDS_ADDR_CONFLICT")


def pmc_sequence(configs, dev):
    """(op name, zero-arg launcher) in the order `--pmc-driver` dispatches them."""
    import comfy_kitchen as ck

    seq = []
    if "c1" in configs:
        x, scale = make_c1(dev)
        q = ck.quantize_per_tensor_fp8(x, scale)
        seq += [("quantize_per_tensor_fp8", lambda: ck.quantize_per_tensor_fp8(x, scale)),
                ("dequantize_per_tensor_fp8", lambda: ck.dequantize_per_tensor_fp8(q, scale))]
    if "c2" in configs:
        qq, kk, f = make_c2(dev)
        seq += [("apply_rope", lambda: ck.apply_rope(qq, kk, f)), ("apply_rope1", lambda: ck.apply_rope1(qq, f))]
    if "c3" in configs or "c4" in configs:
        x3 = make_c3(dev)
        qa, sa = ck.quantize_mxfp8(x3)
        if "c3" in configs:
            seq += [("quantize_mxfp8", lambda: ck.quantize_mxfp8(x3)),
                    ("dequantize_mxfp8", lambda: ck.dequantize_mxfp8(qa, sa))]
        if "c4" in configs:
            qw, sw = ck.quantize_mxfp8(make_c4_weight(dev))
            seq.append(("scaled_mm_mxfp8", lambda: ck.scaled_mm_mxfp8(qa, qw, sa, sw)))
    if "c5" in configs:
        a, w, ga, gw = make_c5(dev)
        na, nsa = ck.quantize_nvfp4(a, ga)
        nw, nsw = ck.quantize_nvfp4(w, gw)
        seq += [("quantize_nvfp4", lambda: ck.quantize_nvfp4(a, ga)),
                ("dequantize_nvfp4", lambda: ck.dequantize_nvfp4(na, ga, nsa)),
                ("scaled_mm_nvfp4", lambda: ck.scaled_mm_nvfp4(na, nw, ga, gw, nsa, nsw))]
    # --summarize-pmc walks the counter rows in the order pmc_sequence_names gives
    assert [n for n, _ in seq] == [n for n, _ in pmc_sequence_names(configs)], "PMC sequence and names disagree"
    return seq


def pmc_driver(configs):
    """The MFMA-busy calibration loop (one workgroup per CU), one traffic calibration kernel
    (negate 256 MiB of fp32: reads and writes PMC_CALIB_BYTES), then PMC_CALLS eager calls
    of each op; no hipMemset/copy between them."""
    dev = torch.device("cuda", 0)
    seq = pmc_sequence(configs, dev)
    src = torch.ones(PMC_CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cus * 256, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    assert bench_lib().ckh_bench_mfma_loop(sink.data_ptr(), cus, PMC_MFMA_ITERS,
                                           torch.cuda.current_stream().cuda_stream) == 0
    torch.neg(src, out=dst)
    for _, fn in seq:
        for _ in range(PMC_CALLS):
            fn()
    torch.cuda.synchronize()
    print(json.dumps({"pmc_sequence": [n for n, _ in seq], "calls": PMC_CALLS}), flush=True)


def _pmc_dispatches(d: Path, counter: str):
    """[(dispatch id, kernel name, value)] of one counter from a rocprofv3 --pmc csv directory."""
    import csv

    rows = []
    for f in sorted(d.rglob("*counter_collection.csv")):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


# kernel-name substring of each op's own dispatches (an op may launch several per call)
OP_KERNELS = {"quantize_per_tensor_fp8": "ckh::quantize_fp8", "dequantize_per_tensor_fp8": "ckh::dequantize_fp8",
              "apply_rope": "ckh::rope", "apply_rope1": "ckh::rope", "quantize_mxfp8": "ckh::quantize_mxfp8",
              "dequantize_mxfp8": "ckh::dequantize_mxfp8", "scaled_mm_mxfp8": "ckh::mx::gemm",
              "quantize_nvfp4": "ckh::quantize_nvfp4", "dequantize_nvfp4": "ckh::dequantize_nvfp4",
              "scaled_mm_nvfp4": "ckh::nv::gemm"}


def summarize_pmc(fetch_dir: str, write_dir: str, configs, command: str):
    """L2-miss bytes per launch of each op: counter KiB scaled by calibration bytes / calibration KiB."""
    seq = [n for n, _ in pmc_sequence_names(configs)]
    out = {"what": "bytes per launch that missed L2 (TCC FETCH_SIZE, WRITE_SIZE): HBM traffic plus Infinity-Cache "
                   "hits, an upper bound on HBM bytes", "bytes_per_launch": {}, "calibration": {}, "command": command}
    for key, d, counter in (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        rows = _pmc_dispatches(Path(d), counter)
        # calibration: the largest non-ckh dispatch; the measured sequence follows it
        ci = max((i for i, r in enumerate(rows) if "ckh::" not in r[1]), key=lambda i: rows[i][2])
        calib = rows[ci]
        factor = PMC_CALIB_BYTES / (calib[2] * 1024.0)
        out["calibration"][counter] = {"kernel": calib[1][:60], "kib": calib[2], "factor": round(factor, 4)}
        ours = [r for r in rows[ci + 1:] if "ckh::" in r[1]]  # the ops' own kernels, in order
        i = 0
        for name in seq:
            sub, run = OP_KERNELS[name], []
            # apply_rope and apply_rope1 share a kernel (one dispatch per call each)
            cap = PMC_CALLS if name.startswith("apply_rope") else len(ours)
            while i < len(ours) and sub in ours[i][1] and len(run) < cap:
                run.append(ours[i][2])
                i += 1
            assert run, f"no dispatches of {name} in the counter run"
            b = sum(run) / PMC_CALLS * 1024.0 * factor
            out["bytes_per_launch"].setdefault(name, {})[key] = round(b)
            out["bytes_per_launch"][name]["dispatches_per_call"] = len(run) // PMC_CALLS
    for name, v in out["bytes_per_launch"].items():
        v["total"] = v.get("fetch", 0) + v.get("write", 0)
    (REPO / "profiles").mkdir(exist_ok=True)
    (REPO / "profiles" / "traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))


def summarize_counters(sq_dir: str, configs, command: str):
    """MFMA busy and LDS conflicts per op from one rocprofv3 --pmc pass over SQ_COUNTERS.

    MFMA busy = (SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES) of the op's dispatch divided by
    the same ratio of the calibration loop, which keeps every SIMD's matrix core busy (the
    MFMA counter sums over SIMDs, SQ_BUSY_CYCLES over shader engines).  Writes
    profiles/counters.json and prints a markdown table."""
    import csv

    disp = {}
    for f in sorted(Path(sq_dir).rglob("*counter_collection.csv")):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                e = disp.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], {}])
                e[1][r["Counter_Name"]] = e[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    rows = [(i, *disp[i]) for i in sorted(disp)]
    ci = next(i for i, r in enumerate(rows) if "mfma_loop_kernel" in r[1])
    cal = rows[ci][2]
    full = cal["SQ_VALU_MFMA_BUSY_CYCLES"] / cal["SQ_BUSY_CYCLES"]
    ours = [r for r in rows[ci + 1:] if "ckh::" in r[1]]
    out = {"command": command, "calibration": {"kernel": rows[ci][1][:60], "mfma_busy_per_sq_busy": round(full, 3)},
           "ops": {}}
    i = 0
    for name, _ in pmc_sequence_names(configs):
        sub, run = OP_KERNELS[name], []
        cap = PMC_CALLS if name.startswith("apply_rope") else len(ours)
        while i < len(ours) and sub in ours[i][1] and len(run) < cap:
            run.append(ours[i])
            i += 1
        assert run, f"no dispatches of {name} in the counter run"
        kern = {}
        for _, k, c in run:
            acc = kern.setdefault(k, {"n": 0})
            acc["n"] += 1
            for cn, v in c.items():
                acc[cn] = acc.get(cn, 0.0) + v
        for k, acc in kern.items():
            n = acc.pop("n")
            mean = {cn: v / n for cn, v in acc.items()}
            lds = max(mean.get("SQ_INSTS_LDS", 0.0), 1.0)
            out["ops"].setdefault(name, []).append({
                "kernel": k[:80], "dispatches": n,
                "mfma_busy": round(mean["SQ_VALU_MFMA_BUSY_CYCLES"] / mean["SQ_BUSY_CYCLES"] / full, 4),
                "lds_bank_conflict_cycles_per_lds_inst": round(mean.get("SQ_LDS_BANK_CONFLICT", 0.0) / lds, 4),
                "valu_insts_per_mfma": (round(mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"], 2)
                                        if mean.get("SQ_INSTS_MFMA") else None),
                **{cn: round(v) for cn, v in sorted(mean.items())}})
    (REPO / "profiles").mkdir(exist_ok=True)
    (REPO / "profiles" / "counters.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"calibration ({out['calibration']['kernel']}): SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES = {full:.3f}")
    print("| op | kernel | MFMA busy | LDS bank-conflict cycles | LDS address conflicts | LDS insts | MFMA insts | "
          "VALU insts per MFMA |")
    print("|---|---|---|---|---|---|---|---|")
    for name, ks in out["ops"].items():
        for e in ks:
            has_mfma = e["valu_insts_per_mfma"] is not None
            busy = f"{100 * e['mfma_busy']:.1f}%" if has_mfma else "-"
            ratio = e["valu_insts_per_mfma"] if has_mfma else "-"
            print(f"| {name} | `{e['kernel'][:48]}` | {busy} | {e.get('SQ_LDS_BANK_CONFLICT', 0):,} | "
                  f"{e.get('SQ_LDS_ADDR_CONFLICT', 0):,} | {e.get('SQ_INSTS_LDS', 0):,} | {e.get('SQ_INSTS_MFMA', 0):,} | "
                  f"{ratio} |")


# (config, kernel-name substring of the op's timed kernel, algorithmic units) per op, for the
# per-op profile summaries
PROFILE_OPS = {
    "quantize_per_tensor_fp8": ("c1", "quantize_fp8_pipe_kernel<2, 5>"),
    "dequantize_per_tensor_fp8": ("c1", "dequantize_fp8_kernel<5, 2, true>"),
    "apply_rope": ("c2", "rope_wave_kernel<2, 0, false>"),
    "apply_rope1": ("c2", "rope_wave_kernel<2, 0, true>"),
    "quantize_mxfp8": ("c3", "quantize_mxfp8_fast_kernel<2>"),
    "dequantize_mxfp8": ("c3", "dequantize_mxfp8_fast_kernel<2>"),
    "scaled_mm_mxfp8": ("c4", "mx::gemm_kernel<2, -1, false>"),
    "quantize_nvfp4": ("c5", "quantize_nvfp4_fast_kernel<2, true, 16, false>"),
    "dequantize_nvfp4": ("c5", "dequantize_nvfp4_tile_kernel<2, true>"),
    "scaled_mm_nvfp4": ("c5", "nv::gemm_kernel<2, -1>"),
}


def summarize_trace(kt_dir: str, bench_json: str, command: str):
    """profiles/<op>_<config>.md from a rocprofv3 --kernel-trace run of bench.py (graph-replay
    dispatches: runs of >= 20 back-to-back dispatches of the op's kernel), the bench line of
    a run without the profiler, profiles/traffic.json and profiles/counters.json."""
    import csv
    import statistics

    rows = []
    for f in sorted(Path(kt_dir).rglob("*kernel_trace.csv")):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    line = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
    prof = REPO / "profiles"
    traffic = json.loads((prof / "traffic.json").read_text()) if (prof / "traffic.json").exists() else {}
    counters = json.loads((prof / "counters.json").read_text()) if (prof / "counters.json").exists() else {}
    for op, (cfg, sub) in PROFILE_OPS.items():
        res = line["ops"].get(op)
        if res is None or "ms" not in res:
            continue
        # the op's dispatches, grouped into runs separated by more than 20 us (or 5% of a
        # dispatch) of idle time: an op may launch a small kernel of its own in between
        # (the NVFP4 GEMM's alpha product), so other kernels do not split a run
        mine = [(s0, e0, k) for s0, e0, k in rows if sub in k]
        durs, run = [], []
        for d in mine:
            if run and d[0] - run[-1][1] > max(20000, (run[-1][1] - run[-1][0]) // 20):
                if len(run) >= 20:
                    durs += [(e0 - s0) / 1e3 for s0, e0, _ in run]
                run = []
            run.append(d)
        if len(run) >= 20:
            durs += [(e0 - s0) / 1e3 for s0, e0, _ in run]
        name = mine[0][2] if mine else ""
        if not durs:
            continue
        us = res["ms"] * 1e3
        out = [f"# {op} — BASELINE {cfg}", "",
               "Kernel durations from the kernel trace of a bench run, over the op's HIP-graph replays (runs of",
               "back-to-back dispatches of its kernel: the settle replays and the five timed rounds):", "",
               f"    {command}", "",
               "| kernel | dispatches | mean µs | median µs | min µs | max µs |", "|---|---|---|---|---|---|",
               f"| `{name[:110]}` | {len(durs)} | {statistics.mean(durs):.2f} | {statistics.median(durs):.2f} | "
               f"{min(durs):.2f} | {max(durs):.2f} |", "",
               f"bench.py without the profiler (`python -u bench.py`, median of five graph replays of K calls between "
               f"HIP events on the launch stream): **{us:.2f} µs** per call → {res['achieved']} {res['unit']} = "
               f"{100 * res['frac']:.1f}% of {res['peak']} {res['unit']}."]
        if "copy_floor_ms" in res:
            out += ["", f"Copy floor for the same bytes in the same run (`benchlib/copy_floor.hip`, timed in alternating "
                        f"rounds with the op): {res['copy_floor_ms'] * 1e3:.2f} µs; the op runs at "
                        f"{100 * res['of_copy_floor']:.1f}% of it."]
        t = traffic.get("bytes_per_launch", {}).get(op)
        if t:
            cal = traffic.get("calibration", {})
            out += ["", "L2-miss bytes per launch, i.e. HBM traffic plus Infinity-Cache hits (rocprofv3 `--pmc "
                        "FETCH_SIZE`, then `--pmc WRITE_SIZE`, over `python -u bench.py --pmc-driver`, three eager "
                        "calls on the same buffers, scaled by a 256 MiB calibration kernel: FETCH "
                        f"×{cal.get('FETCH_SIZE', {}).get('factor', '?')}, WRITE ×{cal.get('WRITE_SIZE', {}).get('factor', '?')}):",
                    "", "| fetched B | written B | total B |", "|---|---|---|",
                    f"| {t.get('fetch', 0):,} | {t.get('write', 0):,} | {t.get('total', 0):,} |"]
        c = counters.get("ops", {}).get(op)
        if c and c[0].get("valu_insts_per_mfma") is not None:
            e = c[0]
            out += ["", "## MFMA busy and LDS conflicts (SQ counters, one pass; `profiles/counters.json`)", "",
                    f"    {counters.get('command', '')}", "",
                    "MFMA busy = (SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES) of the GEMM's dispatch ÷ the same ratio of "
                    "a calibration loop of back-to-back MFMAs on every SIMD (`benchlib/mfma_loop.hip`, "
                    f"{counters['calibration']['mfma_busy_per_sq_busy']}), averaged over {e['dispatches']} eager calls "
                    "on the same operands.", "",
                    "| kernel | MFMA busy | MFMA insts | LDS insts | LDS bank-conflict cycles | per LDS inst | "
                    "LDS address conflicts | VALU insts per MFMA |", "|---|---|---|---|---|---|---|---|",
                    f"| `{e['kernel']}` | {100 * e['mfma_busy']:.1f}% | {e['SQ_INSTS_MFMA']:,} | {e['SQ_INSTS_LDS']:,} | "
                    f"{e['SQ_LDS_BANK_CONFLICT']:,} | {e['lds_bank_conflict_cycles_per_lds_inst']} | "
                    f"{e['SQ_LDS_ADDR_CONFLICT']:,} | {e['valu_insts_per_mfma']} |"]
        (prof / f"{op}_{cfg}.md").write_text("\n".join(out) + "\n")
        print(f"wrote profiles/{op}_{cfg}.md ({len(durs)} dispatches, mean {statistics.mean(durs):.2f} us, "
              f"bench {us:.2f} us)")


# C4 GEMMs side by side with the vendor's: `--pmc-gemm-driver` dispatches the MFMA-loop
# calibration, the 256 MiB traffic calibration, then PMC_CALLS calls each of
# ck.scaled_mm_mxfp8, ck.scaled_mm_fp8 (unit scales), torch._scaled_mm tensor-wise and
# torch's F.scaled_mm with 1 x 32 E8M0 scales on the C4 operands; `--summarize-gemm` joins a
# kernel-trace run, an SQ-counter run and a FETCH_SIZE run of it into
# profiles/scaled_mm_c4_vs_vendor.md.
GEMM_OPS = ("ck.scaled_mm_mxfp8", "ck.scaled_mm_fp8", "torch._scaled_mm tensor-wise",
            "F.scaled_mm BlockWise1x32 (row-major E8M0)")


def pmc_gemm_driver():
    import torch.nn.functional as F

    import comfy_kitchen as ck

    dev = torch.device("cuda", 0)
    qa, sa = ck.quantize_mxfp8(make_c3(dev))
    qw, sw = ck.quantize_mxfp8(make_c4_weight(dev))
    m, k = qa.shape
    n = qw.shape[0]
    one = torch.ones(1, device=dev)
    sa_p = ck.from_blocked(sa.view(torch.uint8), m, k // 32).contiguous().view(torch.float8_e8m0fnu)
    sw_p = ck.from_blocked(sw.view(torch.uint8), n, k // 32).contiguous().view(torch.float8_e8m0fnu)
    calls = [lambda: ck.scaled_mm_mxfp8(qa, qw, sa, sw), lambda: ck.scaled_mm_fp8(qa, qw, one, one),
             lambda: torch._scaled_mm(qa, qw.t(), one.reshape(()), one.reshape(()), out_dtype=torch.bfloat16),
             # the swizzle arguments must be given: torch 2.10 on ROCm dereferences a null
             # pointer on the host when they are left out
             lambda: F.scaled_mm(qa, qw.t(), scale_a=sa_p, scale_recipe_a=F.ScalingType.BlockWise1x32, scale_b=sw_p,
                                 scale_recipe_b=F.ScalingType.BlockWise1x32, swizzle_a=F.SwizzleType.NO_SWIZZLE,
                                 swizzle_b=F.SwizzleType.NO_SWIZZLE, output_dtype=torch.bfloat16)]
    for c in calls:  # warm up outside the counted sequence order (the summary matches by name)
        c()
    src = torch.ones(PMC_CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cus * 256, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    assert bench_lib().ckh_bench_mfma_loop(sink.data_ptr(), cus, PMC_MFMA_ITERS,
                                           torch.cuda.current_stream().cuda_stream) == 0
    torch.neg(src, out=dst)
    for c in calls:
        for _ in range(PMC_CALLS):
            c()
    torch.cuda.synchronize()
    print(json.dumps({"gemm_sequence": GEMM_OPS, "calls": PMC_CALLS}), flush=True)


def summarize_gemm(kt_dir: str, sq_dir: str, fetch_dir: str, command: str):
    """profiles/scaled_mm_c4_vs_vendor.md (+ .json): per GEMM kernel of the --pmc-gemm-driver
    sequence, its duration (kernel trace), the clock its SQ_BUSY_CYCLES imply over that
    duration, MFMA busy, instruction mix, LDS conflicts and L2-miss fetch bytes."""
    import csv
    import statistics

    def rows(d, fname):
        out = []
        for f in sorted(Path(d).rglob(fname)):
            with open(f) as fh:
                out += list(csv.DictReader(fh))
        return out

    kt = sorted(rows(kt_dir, "*kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    dur = {}
    for r in kt:
        dur.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)

    def per_dispatch(d):
        disp = {}
        for r in rows(d, "*counter_collection.csv"):
            e = disp.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], {}])
            e[1][r["Counter_Name"]] = e[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        return [disp[i] for i in sorted(disp)]

    sq, fe = per_dispatch(sq_dir), per_dispatch(fetch_dir)
    cal = next(c for name, c in sq if "mfma_loop_kernel" in name)
    cal_name = next(name for name, _ in sq if "mfma_loop_kernel" in name)
    full = cal["SQ_VALU_MFMA_BUSY_CYCLES"] / cal["SQ_BUSY_CYCLES"]
    # the calibration loop: PMC_MFMA_ITERS x 16 MFMAs of 64 cycles per wave, all SIMDs busy
    cal_cycles = PMC_MFMA_ITERS * 16 * 64
    n_se = cal["SQ_BUSY_CYCLES"] / cal_cycles
    cal_us = statistics.median(dur.get(cal_name, [float("nan")]))
    fcal = max((c["FETCH_SIZE"], name) for name, c in fe if "mfma_loop" not in name and "ckh::" not in name
               and "gemm" not in name.lower() and "Cijk" not in name)
    fscale = PMC_CALIB_BYTES / (fcal[0] * 1024.0)
    gemm = lambda name: ("ckh::" in name and "gemm" in name) or "Cijk" in name or "GEMM" in name  # noqa: E731
    table = {}
    for name, c in sq:
        if gemm(name):
            table.setdefault(name, {"sq": [], "fetch": []})["sq"].append(c)
    for name, c in fe:
        if name in table:
            table[name]["fetch"].append(c["FETCH_SIZE"] * 1024.0 * fscale)
    out = {"command": command, "calibration": {"kernel": cal_name[:60], "mfma_busy_per_sq_busy": round(full, 3),
                                               "shader_engines": round(n_se, 2), "median_us": round(cal_us, 2),
                                               "clock_ghz": round(cal_cycles / cal_us / 1e3, 3)},
           "kernels": {}}
    lines = ["# C4 GEMMs against the vendor's (hipBLASLt through torch) — counters side by side", "",
             "Sequence (`python3 -u bench.py --pmc-gemm-driver`): the MFMA-loop calibration, a 256 MiB negate "
             "(traffic calibration), then three calls each of " + ", ".join(f"`{o}`" for o in GEMM_OPS) +
             " on the C4 operands (A [4608, 3072], B [12288, 3072], bf16 out).", "",
             "Commands (each a run of its own):", "", *[f"    {c.strip()}" for c in command.split(";") if c.strip()], "",
             "- implied clock = SQ_BUSY_CYCLES / shader engines / duration (shader engines from the calibration "
             f"loop, whose MFMA cycles are known: {n_se:.2f}); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES "
             f"÷ the calibration's ratio ({full:.3f});",
             "- fetch = TCC FETCH_SIZE scaled by the traffic calibration: bytes that missed L2 (HBM + MALL).", "",
             "| kernel | calls | mean µs | implied clock GHz | MFMA busy | MFMA insts | LDS insts | LDS bank-conflict "
             "cycles | VALU insts / MFMA | fetch MB |", "|---|---|---|---|---|---|---|---|---|---|"]
    for name, e in table.items():
        mean = {cn: statistics.mean(c[cn] for c in e["sq"]) for cn in e["sq"][0]}
        us = statistics.mean(dur.get(name, [float("nan")])[-PMC_CALLS:])
        clock = mean["SQ_BUSY_CYCLES"] / n_se / us / 1e3
        busy = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / mean["SQ_BUSY_CYCLES"] / full
        vpm = mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"] if mean.get("SQ_INSTS_MFMA") else float("nan")
        fetch = statistics.mean(e["fetch"]) / 1e6 if e["fetch"] else float("nan")
        out["kernels"][name] = {"calls": len(e["sq"]), "mean_us": round(us, 2), "clock_ghz": round(clock, 3),
                                "mfma_busy": round(busy, 4), "valu_per_mfma": round(vpm, 2),
                                "fetch_bytes": round(fetch * 1e6), **{cn: round(v) for cn, v in sorted(mean.items())}}
        lines.append(f"| `{name[:90]}` | {len(e['sq'])} | {us:.1f} | {clock:.2f} | {100 * busy:.1f}% | "
                     f"{mean['SQ_INSTS_MFMA']:,.0f} | {mean['SQ_INSTS_LDS']:,.0f} | {mean['SQ_LDS_BANK_CONFLICT']:,.0f} | "
                     f"{vpm:.2f} | {fetch:.1f} |")
    prof = REPO / "profiles"
    prof.mkdir(exist_ok=True)
    (prof / "scaled_mm_c4_vs_vendor.md").write_text("\n".join(lines) + "\n")
    (prof / "scaled_mm_c4_vs_vendor.json").write_text(json.dumps(out, indent=1) + "\n")
    print("\n".join(lines))


def pmc_sequence_names(configs):
    names = []
    if "c1" in configs:
        names += ["quantize_per_tensor_fp8", "dequantize_per_tensor_fp8"]
    if "c2" in configs:
        names += ["apply_rope", "apply_rope1"]
    if "c3" in configs:
        names += ["quantize_mxfp8", "dequantize_mxfp8"]
    if "c4" in configs:
        names.append("scaled_mm_mxfp8")
    if "c5" in configs:
        names += ["quantize_nvfp4", "dequantize_nvfp4", "scaled_mm_nvfp4"]
    return [(n, None) for n in names]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5,lin,sweep",
                    help="BASELINE configs c1..c5, lin (Flux/Wan linear shapes), sweep (copy size sweep)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc-driver", action="store_true", help="dispatch sequence for rocprofv3 --pmc passes")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic.json from two rocprofv3 --pmc output directories")
    ap.add_argument("--pmc-command", default="", help="command recorded in profiles/traffic.json")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("KT_DIR", "BENCH_JSON"),
                    help="write profiles/<op>_<config>.md from a rocprofv3 --kernel-trace run and a bench line")
    ap.add_argument("--pmc-gemm-driver", action="store_true",
                    help="C4 GEMM sequence (ours and the vendor's) for rocprofv3 passes")
    ap.add_argument("--summarize-gemm", nargs=3, metavar=("KT_DIR", "SQ_DIR", "FETCH_DIR"),
                    help="write profiles/scaled_mm_c4_vs_vendor.md from runs of --pmc-gemm-driver")
    ap.add_argument("--summarize-counters", metavar="SQ_DIR",
                    help="write profiles/counters.json (MFMA busy, LDS conflicts) from a rocprofv3 --pmc pass "
                         "over SQ_COUNTERS")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc, set(args.configs.split(",")), args.pmc_command)
        return
    if args.summarize_counters:
        summarize_counters(args.summarize_counters, set(args.configs.split(",")), args.pmc_command)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace, args.pmc_command)
        return
    if args.summarize_gemm:
        summarize_gemm(*args.summarize_gemm, args.pmc_command)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the quantizers and GEMMs would shard by rows with no exchange between GPUs).", file=sys.stderr)
        sys.exit(2)
    configs = set(args.configs.split(","))

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    import comfy_kitchen as ck

    if not ck.list_backends()["hip"]["available"]:
        sys.exit(f"hip backend unavailable: {ck.list_backends()['hip']['unavailable_reason']}")
    if args.pmc_driver:
        pmc_driver(configs)
        return
    if args.pmc_gemm_driver:
        pmc_gemm_driver()
        return
    gpu = run_gpu(configs, args.steps, args.warmup, log)
    if "lin" in configs:
        gpu["linear_shapes"] = run_linear_shapes(args.steps, args.warmup, log)
        gpu["nv_linear_shapes"] = run_nv_linear_shapes(args.steps, args.warmup, log)
    sweep = run_copy_sweep(log) if "sweep" in configs else None
    cpu = {} if args.no_cpu else run_cpu_baseline(configs, log)

    # the headline op: quantize_mxfp8 (config 3), else the first op measured with a roofline
    with_roof = [k for k, v in gpu.items() if isinstance(v, dict) and "bound" in v]
    if not with_roof:
        print(json.dumps({"metric": METRIC, "ops": gpu, "copy_sweep": sweep, "note": "no roofline op in --configs"}),
              flush=True)
        return
    primary = "quantize_mxfp8" if "quantize_mxfp8" in gpu else with_roof[0]
    p = gpu[primary]
    roof = {k: p[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")}
    roof["traffic_counts"] = "L2-miss bytes per launch (TCC FETCH_SIZE + WRITE_SIZE): HBM plus Infinity-Cache hits"
    line = {
        "metric": METRIC,
        "value": p["achieved"],
        "unit": p["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(p["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16->e4m3/e8m0",
        "data": "synthetic (seeded; BASELINE.json config shapes and distributions)",
        "config": {"workload": f"{primary} (BASELINE config 3: bf16 [4608, 3072], per-row log-normal)",
                   "timing": "HIP graph of K calls, rotating >512MB of buffers, HIP events on the launch stream"},
        "roofline": roof,
        "cpu_baseline": cpu.get(primary),
        "ops": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()} for k, v in gpu.items()},
        "cpu_baselines": cpu,
        "copy_sweep": sweep,
        "device": torch.cuda.get_device_properties(0).gcnArchName,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
