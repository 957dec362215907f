#!/usr/bin/env python3
"""Expert-FFN decode benchmark on one MI355X (BASELINE.json metric).

Workload (default, configs[1] = C2): GPT-OSS-20B-shape 24-layer MoE expert stack
(hidden 2880, 32 MXFP4 experts per layer, top-4, intermediate 2880), batch-1
decode. One step = one token through all 24 layers (router -> top-k -> gate/up
+ SwiGLU -> down + weighted combine per layer), layer-serial in stream order.
Weights are synthetic (seeded, generated on the GPU), all resident in HBM.

Prints ONE JSON line. `value` is tokens/s over the K timed steps (inputs already
resident in HBM). `roofline` is the dominant kernel's algorithmic bytes per
launch over its average launch duration, measured with HIP events on the
library's stream. `cpu_baseline` times the CPU oracle (the C restatement of the
reference's CPU path) on a bounded sample on this host. `extra_configs` (default run
only) holds the same measurement, with fewer steps and no CPU leg, for C1, C2 chained through the
fused norm and residual, C3 and C4 (decode) and C5 (batched): value, unit, dominant kernel, its
average launch and its roofline fraction.
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
sys.path.insert(0, str(ROOT / "moe-stream_amd"))

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--kernel", default="auto", choices=["auto", "valu", "fused"])
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--residual", action="store_true",
                    help="time mr_moe_forward_residual (post-attention RMSNorm + MoE + residual add)")
    ap.add_argument("--batched", type=int, default=0,
                    help="time mr_moe_forward_batched on layer 0 of --config with this many tokens "
                         "(C5 is always a batched run, of 512 tokens unless this is given)")
    ap.add_argument("--decode", default="layers", choices=["layers", "chain"],
                    help="layers: every layer reads its own input x[token][layer] (mr_moe_forward); "
                         "chain: one hidden state per token carried through the layers in place, one "
                         "mr_moe_forward_residual per layer")
    ap.add_argument("--no-prefetch-hint", action="store_true",
                    help="do not link each layer to the next (mr_layer_set_next)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="headline only: skip the C1, C2-chained, C3, C4 and C5 rows of extra_configs")
    ap.add_argument("--profile-tokens", type=int, default=16)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle threads for the CPU baseline (0: every logical core, as the reference's available_parallelism)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain copy kernel of known size (counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--trace", action="store_true",
                    help="only trace one fused MXFP4 decode launch (layer 5 of a token, --config 1 or 2) with the "
                         "library built by `python moe-stream_amd/moe_rocm/build.py --trace`: phase times per role")
    ap.add_argument("--trace-graph", action="store_true",
                    help="with --trace: trace two consecutive layers inside a replayed token graph (the timed "
                         "pipeline's conditions), and the gap between them")
    ap.add_argument("--probe", action="store_true",
                    help="only measure the ceilings: a graph of empty kernels (the kernel-boundary floor) and "
                         "plain streaming reads of the decode layers' byte counts")
    ap.add_argument("--probe-flags", action="store_true",
                    help="only measure flag round trips between two workgroups (within one XCD and across XCDs)")
    ap.add_argument("--probe-eager", action="store_true",
                    help="the plain reads of --probe launched one at a time (512 workgroups, 8 loads in flight), "
                         "for a kernel trace (rocprofv3 --kernel-trace) of their device durations")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(layers, specs, threads: int, budget_s: float = 12.0):
    """The oracle (C restatement of the reference CPU path) on a bounded sample of the
    workload: the same N decode tokens through every layer of the stack, one layer's
    weights on the host at a time, with N sized from a one-token calibration on the first
    layer so that the sample takes about budget_s of CPU work. A token's time is the sum
    of its layers' times, so tokens/s = N / (total time). Returns (tokens/s, N, seconds)."""
    import oracle  # test infrastructure; used here only as the timed CPU baseline
    from moe_rocm import workloads as W

    n_tok, total = None, 0.0
    for dl, spec in zip(layers, specs):
        host = dict(spec=spec)
        host.update(dl.download_quant())
        host.update(W.float_tensors(spec))
        L = oracle.layer_from_host(host)
        if n_tok is None:
            x1 = W.x_tokens(spec, 1)
            L.forward(x1, n_threads=threads)  # warm-up
            t0 = time.perf_counter()
            L.forward(x1, n_threads=threads)
            n_tok = max(1, int(budget_s / (len(specs) * (time.perf_counter() - t0))))
        x = W.x_tokens(spec, n_tok)
        t0 = time.perf_counter()
        for t in range(n_tok):
            L.forward(x[t:t + 1], n_threads=threads)
        total += time.perf_counter() - t0
        del host, L
    return n_tok / total, n_tok, total


def copy_calibration(n_bytes: int = 1 << 30, reps: int = 4) -> None:
    """A plain streaming kernel of known traffic: reads n_bytes, writes n_bytes
    per dispatch (torch elementwise multiply on float32). Under rocprofv3 --pmc,
    FETCH_SIZE / WRITE_SIZE of this kernel over n_bytes is the counter's scale."""
    import torch

    a = torch.ones(n_bytes // 4, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(reps):
        torch.mul(a, 2.0, out=b)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"read_bytes": n_bytes, "write_bytes": n_bytes,
                                           "dispatches": reps, "kernel": "torch mul float32"}}))


def probes() -> None:
    """Ceilings of the decode path on this GPU, with the library's probe kernels, every
    launch inside a HIP graph as in the timed decode:
    - kernel boundary: a graph of 24 empty kernels (a token's graph holds 24 layer launches)
      with the C2 fused kernel's grid and with one workgroup, time per kernel;
    - plain stream: mr_probe_read (each workgroup a contiguous range, 4, 8 or 16 16-byte loads
      in flight per thread) over byte counts from 2.2 MB to 214 MB, among them one C2 layer's
      53.4 MB, its gate/up weights' 35.2 MB and one C3 layer's 22.3 MB, with 256 to 2048
      workgroups. One graph holds n launches reading consecutive regions of a 1.5 GiB pool
      (n x bytes >= 768 MB, beyond the 256 MB Infinity Cache), so every byte comes from HBM.
      Per (grid, depth): the least-squares fit t = t0 + bytes / B over the sizes, which splits a
      launch into its fixed cost t0 (launch in the graph, ramp, first-touch latency, drain) and
      the sustained rate B; and a 1 GiB read per launch as a check of B."""
    import moe_rocm as M
    from moe_rocm import workloads as W

    ctx = M.Context(0)
    c2 = W.gpt_oss(2, 0)
    c2_bytes, c3_bytes = c2.weight_bytes_per_token(), W.qwen3_30b(3, 0).weight_bytes_per_token()
    gu_bytes = c2.top_k * 2 * M.synth.matrix_bytes(c2.ggml_type, c2.inter, c2.hidden)
    fused_grid = 576  # C2 fused kernel
    out = {"probe": "decode ceilings", "method": "HIP graphs; event time over the graph / launches"}
    floor = {}
    for n_wg in (fused_grid, 1):
        ctx.graph_begin()
        for _ in range(24):
            ctx.probe_empty(n_wg)
        g = ctx.graph_end()
        for _ in range(3):
            g.launch()
        ctx.sync()
        reps = 50
        ctx.timer_start()
        for _ in range(reps):
            g.launch()
        ms = ctx.timer_stop()
        g.close()
        floor[str(n_wg)] = round(ms * 1e3 / (reps * 24), 3)
    out["empty_kernel_in_graph_us"] = floor
    pool_bytes = 1536 << 20
    pool = ctx.alloc(pool_bytes)
    ctx.synth_blocks(M.GGML_MXFP4, pool, pool_bytes // 17, 7)
    sink = ctx.alloc(4 * 4096)
    named = {"c2_layer": c2_bytes // 16 * 16, "c2_gate_up": gu_bytes // 16 * 16, "c3_layer": c3_bytes // 16 * 16}
    sizes = sorted(set([s // 16 * 16 for s in (2_200_000, 4_406_400, 8_812_800, 17_625_600, 106_813_696,
                                               213_627_392)] + list(named.values())))
    pts = []
    fits = {}
    for n_wg in (256, 512, 768, 1024, 2048):
        for depth in (4, 8, 16):
            xs, ys = [], []
            for nbytes in sizes:
                n = max(24, -(-(768 << 20) // nbytes))
                stride = (nbytes + 4095) // 4096 * 4096
                n = min(n, (pool_bytes - stride) // stride + 1)
                ctx.graph_begin()
                for i in range(n):
                    ctx.probe_read(pool.ptr + i * stride, nbytes, n_wg, sink, depth=depth)
                g = ctx.graph_end()
                g.launch()
                ctx.sync()
                reps = 3
                ctx.timer_start()
                for _ in range(reps):
                    g.launch()
                ms = ctx.timer_stop()
                g.close()
                us = ms * 1e3 / (reps * n)
                name = next((k for k, v in named.items() if v == nbytes), None)
                pts.append({"workgroups": n_wg, "depth": depth, "nbytes": nbytes, "bytes": name,
                            "launches_per_graph": n, "us": round(us, 3),
                            "GB_per_s": round(nbytes / (us * 1e-6) / 1e9, 1)})
                xs.append(nbytes)
                ys.append(us)
            A = np.vstack([np.ones(len(xs)), np.asarray(xs, np.float64)]).T
            (t0, inv_b), *_ = np.linalg.lstsq(A, np.asarray(ys, np.float64), rcond=None)
            resid = float(np.max(np.abs(A @ np.array([t0, inv_b]) - np.asarray(ys))))
            fits[f"{n_wg}x{depth}"] = {"workgroups": n_wg, "depth": depth, "t0_us": round(float(t0), 3),
                                       "B_GB_per_s": round(1e-3 / inv_b, 1), "max_resid_us": round(resid, 3),
                                       "c2_layer_floor_us": round(float(t0 + inv_b * named["c2_layer"]), 3)}
            log(f"fit {n_wg} wg x depth {depth}: t0 {t0:.2f} us, B {1e-3 / inv_b:.0f} GB/s")
    out["plain_read"] = pts
    out["fit_t0_plus_bytes_over_B"] = fits
    # the gate/up access pattern of the fused MXFP4 kernel over the same bytes as C2's gate/up
    # weights (4 experts x 2 projections x 2880 rows of 1530 bytes = 1440 tiles of 16 rows)
    rb = 1530
    n_tiles = gu_bytes // (16 * rb)
    tile_bytes = n_tiles * 16 * rb
    stride = (tile_bytes + 4095) // 4096 * 4096
    tiles = []
    for n_wg in (256, 512, 768):
        for depth in (2, 4, 8, 0x106, 0x10C, 0x117):
            n = min(max(24, -(-(768 << 20) // tile_bytes)), (pool_bytes - stride) // stride + 1)
            ctx.graph_begin()
            for i in range(n):
                ctx.probe_tiles(pool.ptr + i * stride, rb, n_tiles, n_wg, sink, depth=depth)
            g = ctx.graph_end()
            g.launch()
            ctx.sync()
            ctx.timer_start()
            for _ in range(3):
                g.launch()
            ms = ctx.timer_stop()
            g.close()
            us = ms * 1e3 / (3 * n)
            tiles.append({"workgroups": n_wg, "depth": depth if depth < 0x100 else 1,
                          "chunk_steps": 3 if depth < 0x100 else depth - 0x100, "nbytes": tile_bytes, "us": round(us, 3),
                          "GB_per_s": round(tile_bytes / (us * 1e-6) / 1e9, 1)})
            log(f"tiles {n_wg} wg x depth {depth}: {us:.2f} us, {tile_bytes / (us * 1e-6) / 1e9:.0f} GB/s")
    out["gateup_tile_pattern_read"] = tiles
    big = []
    for n_wg in (1024, 2048):
        for depth in (8, 16):
            nbytes = 1 << 30
            ctx.graph_begin()
            ctx.probe_read(pool.ptr, nbytes, n_wg, sink, depth=depth)
            ctx.probe_read(pool.ptr + (pool_bytes - nbytes) // 4096 * 4096, nbytes, n_wg, sink, depth=depth)
            g = ctx.graph_end()
            g.launch()
            ctx.sync()
            ctx.timer_start()
            for _ in range(3):
                g.launch()
            ms = ctx.timer_stop()
            g.close()
            us = ms * 1e3 / 6
            big.append({"workgroups": n_wg, "depth": depth, "nbytes": nbytes, "us": round(us, 1),
                        "GB_per_s": round(nbytes / (us * 1e-6) / 1e9, 1)})
    out["read_1GiB"] = big
    pool.free(), sink.free()
    ctx.close()
    print(json.dumps(out), flush=True)


def probe_flags() -> None:
    """Round trips of an agent-coherent flag between two workgroups of one launch, the hand-off
    the fused decode kernels use (a stores i, b polls for it and stores i back, a polls for
    that; 2,000 round trips per run, 5 runs per pair). Workgroup b runs on XCD b mod 8: pairs
    (0, 8) and (3, 67) share an XCD, (0, 1) and (0, 4) do not. Device-clock time per round trip,
    with both workgroups' XCC_ID and HW_ID."""
    import moe_rocm as M

    ctx = M.Context(0)
    words, res = ctx.alloc(64 * 4), ctx.alloc(4 * 8)
    n = 2000
    out = {"probe": "flag round trips", "round_trips_per_run": n, "pairs": []}
    for a_, b_ in ((0, 8), (3, 67), (0, 1), (0, 4), (0, 255)):
        runs, ids = [], None
        for _ in range(5):
            ctx.probe_flags(words, a_, b_, n, res)
            ctx.sync()
            r = res.download(np.uint64).astype(np.int64)
            if int(r[1]) != n:
                sys.exit(f"probe_flags: pair {a_},{b_} completed {int(r[1])} of {n} round trips")
            runs.append(float(r[0]) / 100.0 / n)  # 100 MHz clock -> us per round trip
            ids = [{"xcc": int(v) >> 32, "hw_id": hex(int(v) & 0xFFFFFFFF)} for v in (r[2], r[3])]
        out["pairs"].append({"workgroups": [a_, b_], "same_xcd": ids[0]["xcc"] == ids[1]["xcc"], "ids": ids,
                             "us_per_round_trip": {"median": round(float(np.median(runs)), 3),
                                                   "min": round(min(runs), 3), "max": round(max(runs), 3)}})
    print(json.dumps(out), flush=True)
    words.free(), res.free()
    ctx.close()


def probes_eager() -> None:
    """The plain reads of probes() launched eagerly, 20 per size over regions of a 1.5 GiB pool (each
    read from HBM), with 512 workgroups and 8 loads in flight, and the gate/up tile pattern over
    C2's gate/up bytes: under rocprofv3 --kernel-trace each dispatch's device duration is recorded,
    without the graph's launch boundary. Prints the sizes in dispatch order."""
    import moe_rocm as M
    from moe_rocm import workloads as W

    ctx = M.Context(0)
    c2 = W.gpt_oss(2, 0)
    c2_bytes, c3_bytes = c2.weight_bytes_per_token(), W.qwen3_30b(3, 0).weight_bytes_per_token()
    gu_bytes = c2.top_k * 2 * M.synth.matrix_bytes(c2.ggml_type, c2.inter, c2.hidden)
    pool_bytes = 1536 << 20
    pool = ctx.alloc(pool_bytes)
    ctx.synth_blocks(M.GGML_MXFP4, pool, pool_bytes // 17, 7)
    sink = ctx.alloc(4 * 4096)
    sizes = sorted(set([s // 16 * 16 for s in (2_200_000, 4_406_400, 8_812_800, 17_625_600, 106_813_696,
                                               213_627_392, c2_bytes, gu_bytes, c3_bytes)]))
    order = []
    for nbytes in sizes:
        stride = (nbytes + 4095) // 4096 * 4096
        n = (pool_bytes - stride) // stride + 1
        for i in range(20):
            ctx.probe_read(pool.ptr + (i % n) * stride, nbytes, 512, sink, depth=8)
        ctx.sync()
        order.append({"kernel": "probe_read", "nbytes": nbytes, "dispatches": 20})
    rb = 1530
    n_tiles = gu_bytes // (16 * rb)
    stride = (n_tiles * 16 * rb + 4095) // 4096 * 4096
    for i in range(20):
        ctx.probe_tiles(pool.ptr + (i % ((pool_bytes - stride) // stride + 1)) * stride, rb, n_tiles, 512, sink, depth=8)
    ctx.sync()
    order.append({"kernel": "probe_tiles", "nbytes": n_tiles * 16 * rb, "dispatches": 20})
    # translations warmed first: a touch of one word per 4 KiB, 64 KiB or 2 MiB of the region,
    # then the C2 layer's bytes read from it (data still in HBM: the touch reads one line per stride)
    nbytes = c2_bytes // 16 * 16
    stride = (nbytes + 4095) // 4096 * 4096
    n = (pool_bytes - stride) // stride + 1
    for tstride in (0, 4096, 65536, 2 << 20):
        for i in range(20):
            reg = pool.ptr + (i % n) * stride
            if tstride:
                ctx.probe_touch(reg, nbytes, tstride, sink)
            ctx.probe_read(reg, nbytes, 512, sink, depth=8)
        ctx.sync()
        order.append({"kernel": "probe_read", "nbytes": nbytes, "dispatches": 20, "touch_stride": tstride,
                      "interleaved_with": "probe_touch" if tstride else None})
    pool.free(), sink.free()
    ctx.close()
    print(json.dumps({"probe_eager": order, "workgroups": 512, "depth": 8}), flush=True)


def trace_decode(a) -> None:
    """Phase timestamps of one fused decode launch (device clock, 100 MHz, read at each
    role's phase boundaries by thread 0 of every workgroup; the first workgroup start is 0).
    The launch is layer 5 of the seventh token of the bench's layer ring, enqueued eagerly after
    six tokens through every layer, so its router rows were prefetched by layer 4 as in the timed
    pipeline. Also the gate/up workgroups' stream time grouped by how many gate/up and down
    workgroups share their CU (the CU read from the hardware id)."""
    lib = ROOT / "moe-stream_amd" / "moe_rocm" / "trace" / "libmoe_rocm.so"
    os.environ.setdefault("MOE_ROCM_LIB", str(lib))
    import ctypes as C

    import moe_rocm as M
    from moe_rocm import workloads as W

    if not hasattr(M._lib, "mr_debug_fused_trace"):
        sys.exit(f"{M.LIB_PATH} has no trace points: build it with `python moe-stream_amd/moe_rocm/build.py --trace`")
    M._lib.mr_debug_fused_trace.argtypes = [C.c_void_p]
    ctx = M.Context(0)
    specs = W.config_layers(a.config)
    if a.decode == "chain":
        stack = W.ChainStack(ctx, specs)
    else:
        stack = W.DecodeStack(ctx, specs, residual=a.residual)
    stack.load(stack.inputs(8))
    for t in range(6):
        stack.enqueue_token(t)
    li = 5 % len(specs)
    s0 = specs[li]
    if s0.mxfp4:
        # the MXFP4 kernel's router workgroups take rr = 1, 2 or 4 logits each (router_rounds):
        # the fewest that keep routers and down groups in one dispatch round (or, with more than
        # four slots, the grid within three workgroups per CU)
        has_sh = 1 if s0.sh_inter else 0
        ktot = s0.top_k + has_sh
        ND, NG = (s0.hidden + 15) // 16 * ((ktot + 3) // 4), s0.top_k * (s0.inter // 32) + has_sh * (s0.sh_inter // 32)
        n_cu = 256
        rr = next((r for r in (1, 2) if (ktot > 4 or -(-(s0.n_experts + has_sh) // r) + ND < n_cu)
                   and -(-(s0.n_experts + has_sh) // r) + ND + NG <= 3 * n_cu), 4)
        R = -(-(s0.n_experts + has_sh) // rr)
    else:  # Q4_K: the shared expert is one more router row and one more gate/up slot
        has_sh = 1 if s0.sh_inter else 0
        R, ND, NG = (s0.n_experts + has_sh + 3) // 4, s0.hidden // 16, (s0.top_k + has_sh) * (s0.inter // 16)
    buf = ctx.zeros((1024 * 32,), dtype=np.uint64)
    prev = ctx.zeros((1024 * 32,), dtype=np.uint64)  # --trace-graph: the layer before
    def launch(l):
        if a.decode == "chain":
            h = stack.h_ptr(6)
            stack.layers[l].layer.forward_residual(h, stack.d_nw.ptr + l * stack.H * 4, stack.eps, h)
        elif a.residual:
            stack.layers[l].layer.forward_residual(stack.x_ptr(6, l), stack.d_nw.ptr + l * stack.H * 4, stack.eps,
                                                   stack.y_ptr(l))
        else:
            stack.layers[l].layer.forward(stack.x_ptr(6, l), stack.y_ptr(l))

    gap_us = None
    if a.trace_graph:
        # one token through every layer in a graph, as the timed pipeline runs it; the trace
        # pointer is set while layers li-1 and li are captured (their launch arguments keep it)
        li = max(li, 1)
        ctx.sync()
        ctx.graph_begin()
        for l in range(len(specs)):
            M._lib.mr_debug_fused_trace(prev.ptr if l == li - 1 else (buf.ptr if l == li else None))
            launch(l)
        M._lib.mr_debug_fused_trace(None)
        g = ctx.graph_end()
        for _ in range(4):
            g.launch()
        ctx.sync()
        g.close()
        tp = prev.download(np.uint64).reshape(1024, 32).astype(np.int64)
        tb = buf.download(np.uint64).reshape(1024, 32).astype(np.int64)
        np_ = int(np.count_nonzero(tp[:, 0]))
        nb = int(np.count_nonzero(tb[:, 0]))
        gap_us = {"previous_layer_last_exit_to_first_start": round(float(tb[:nb, 0].min() - tp[:np_, 5].max()) / 100.0, 2),
                  "previous_layer_us": round(float(tp[:np_, 5].max() - tp[:np_, 0].min()) / 100.0, 2)}
    else:
        for l in range(li):
            launch(l)
        ctx.sync()
        M._lib.mr_debug_fused_trace(buf.ptr)
        launch(li)
        ctx.sync()
        M._lib.mr_debug_fused_trace(None)
    tr = buf.download(np.uint64).reshape(1024, 32).astype(np.int64)
    grid = int(np.count_nonzero(tr[:, 0]))
    us = (tr[:grid] - tr[:grid, 0].min()) / 100.0
    ridx = np.where(tr[:grid, 6] > 0, tr[:grid, 6] - 1, np.arange(grid))  # role index of each dispatch slot
    role = np.array(["router" if b < R else ("gateup" if R + ND <= b < R + ND + NG else "down") for b in ridx])

    def q(v):
        return {"min": round(float(v.min()), 2), "median": round(float(np.median(v)), 2), "max": round(float(v.max()), 2)}

    phases = {
        "router": {"start": q(us[role == "router", 0]), "logits_published": q(us[role == "router", 1]),
                   "exit": q(us[role == "router", 5])},
        "gateup": {"start": q(us[role == "gateup", 0]), "x_image_built": q(us[role == "gateup", 1]),
                   "routed": q(us[role == "gateup", 2]), "stream_done": q(us[role == "gateup", 3]),
                   "epilogue_stored": q(us[role == "gateup", 4]), "exit": q(us[role == "gateup", 5])},
        "down": {"start": q(us[role == "down", 0]), "routed": q(us[role == "down", 1]),
                 "weights_prepared": q(us[role == "down", 2]), "gateup_count_seen": q(us[role == "down", 3]),
                 "image_in_lds": q(us[role == "down", 4]), "exit": q(us[role == "down", 5])},
    }
    # routing points of the consumer workgroups (slots 8-15, thread 0): poll start, every logit
    # seen, keys formed, top-k selected, state kept
    for rname in ("gateup", "down"):
        raw = tr[:grid][role == rname]
        sel = us[role == rname]
        for slot, name in ((8, "route_poll_start"), (9, "route_logits_seen"), (11, "route_keys"),
                           (13, "route_topk_done"), (15, "route_state_kept")):
            ok = raw[:, slot] != 0
            if ok.any():
                phases[rname][name] = q(sel[ok, slot])
        if raw[:, 10].any():
            phases[rname]["route_polls"] = q(raw[:, 10].astype(np.float64))
    # per-wave points (slots 16-23, where the kernel records them): gate/up dot products done
    # (16 + wave); down dot products done (16 + wave) and combine done (20 + wave)
    for rname in ("gateup", "down"):
        sel = us[role == rname]
        raw = tr[:grid][role == rname]
        for slot, name in ((16, "wave_dots_done"), (20, "wave_combine_done")):
            v = np.concatenate([sel[raw[:, slot + w] != 0, slot + w] for w in range(4)])
            if v.size:
                phases[rname][name] = q(v)
    cu = [(b % 8, int(tr[b, 7])) for b in range(grid)]  # (XCD, hardware CU id); workgroup b runs on XCD b mod 8
    by_cu = {}
    for b in range(grid):
        by_cu.setdefault(cu[b], []).append(b)
    groups = {}
    for b in np.nonzero(role == "gateup")[0]:
        co = by_cu[cu[b]]
        key = f"{sum(role[c] == 'gateup' for c in co)} gateup + {sum(role[c] == 'down' for c in co)} down"
        groups.setdefault(key, []).append(us[b, 3] - us[b, 2])
    out = {"trace": W.CONFIG_NAMES[a.config], "layer": li, "workgroups": grid, "cus": len(by_cu),
           "mode": ("graph, " if a.trace_graph else "eager, ") + ("chain" if a.decode == "chain" else
                                                                   "residual" if a.residual else "layers"),
           "gap": gap_us,
           "kernel_us": round(float(us[:, 5].max()), 2), "phases_us": phases,
           "gateup_stream_us_by_cu_load": {k: {"workgroups": len(v), "median": round(float(np.median(v)), 2),
                                               "max": round(float(max(v)), 2)} for k, v in sorted(groups.items())}}
    print(json.dumps(out), flush=True)
    buf.free(), prev.free()
    stack.close()
    ctx.close()


def measured_traffic(config: int):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel
    calibration), or None when no summary exists for this workload."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    return json.loads(f.read_text()).get(f"C{config}")


def host_cpu() -> dict:
    """Logical core count and model name of this host (/proc/cpuinfo)."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"logical_cores": os.cpu_count(), "model": model}


def output_check(ctx, M, W, stack, y, t_last: int, kernel_opt: int) -> dict:
    """After the timed region: every layer's output of the last timed token, as the token
    graphs left it, against an eager run of the same layer and input through the
    multi-kernel VALU path (another kernel family; each is within 1e-3 of the oracle, so
    the two agree within 2e-3). A layer whose router logits (recomputed in float64 on the
    host) put the k-th and (k+1)-th expert within 1e-5 of the largest logit may route
    differently on the two paths and is reported as tie-ambiguous instead of compared."""
    H = stack.H
    tmp = ctx.alloc(H * 4)
    x_all = stack.d_x.download(np.float32, count=stack.n_layers * H,
                               offset=t_last * stack.n_layers * H * 4).reshape(stack.n_layers, H)
    worst, compared, ambiguous = 0.0, 0, []
    prev = None
    try:
        ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
        for li, dl in enumerate(stack.layers):
            spec = dl.spec
            xp = stack.x_ptr(t_last, li)
            x = x_all[li].astype(np.float64)
            if stack.residual:
                dl.layer.forward_residual(xp, stack.d_nw.ptr + li * H * 4, stack.eps, tmp)
                xin = x / np.sqrt((x * x).mean() + stack.eps) * stack.norm_w[li]
            else:
                dl.layer.forward(xp, tmp)
                xin = x
            ref = tmp.download(np.float32).astype(np.float64)
            rw = dl.f["router_w"].download(np.float32).reshape(spec.n_experts, H).astype(np.float64)
            lg = rw @ xin
            if dl.f["router_b"] is not None:
                lg += dl.f["router_b"].download(np.float32)
            s = np.sort(lg)[::-1]
            if s[spec.top_k - 1] - s[spec.top_k] <= 1e-5 * np.abs(lg).max():
                ambiguous.append(li)
                continue
            moe = ref - x if stack.residual else ref
            err = float(np.abs(y[li] - ref).max() / max(np.abs(moe).max(), 1e-30))
            worst = max(worst, err)
            compared += 1
    finally:
        ctx.set_option(M.OPT_DECODE_KERNEL, kernel_opt)
        tmp.free()
    return {"token": t_last, "layers_compared": compared, "tie_ambiguous_layers": ambiguous,
            "max_rel_err_vs_valu": worst, "tolerance": 2e-3, "pass": bool(compared > 0 and worst <= 2e-3)}


def chain_check(ctx, M, stack, t_last: int, kernel_opt: int) -> dict:
    """After the timed region, for a carried hidden state: the last timed token's chain is
    run again eagerly, one mr_moe_forward_residual per layer with the bench's kernel
    choice, and its final h must be bit-identical to what the timed graphs left. Each layer
    of that eager chain is then checked on its own input against the multi-kernel VALU path,
    relative to the change the layer made to h (tolerance 2e-3, as for independent layers). Errors are not compared across the whole
    chain: with synthetic weights the stack amplifies a 2e-5 difference about 1.5x per
    layer, so two correct kernel families drift apart over 24 layers. A layer whose k-th
    and (k+1)-th router logits (float64 on the host) lie within 1e-5 of the largest is
    tie-ambiguous and not compared."""
    H = stack.H
    h0 = stack.h0[t_last]
    got = stack.outputs()[t_last]
    bf, bv = ctx.alloc(H * 4), ctx.alloc(H * 4)
    worst, compared, ambiguous = 0.0, 0, []
    try:
        bf.upload(h0)
        for li, dl in enumerate(stack.layers):
            spec = dl.spec
            nw = stack.d_nw.ptr + li * H * 4
            hin = bf.download(np.float32)
            ctx.set_option(M.OPT_DECODE_KERNEL, kernel_opt)
            dl.layer.forward_residual(bf, nw, stack.eps, bf)
            ctx.set_option(M.OPT_DECODE_KERNEL, M.DECODE_VALU)
            bv.upload(hin)
            dl.layer.forward_residual(bv, nw, stack.eps, bv)
            x = hin.astype(np.float64)
            xin = x / np.sqrt((x * x).mean() + stack.eps) * stack.norm_w[li]
            rw = dl.f["router_w"].download(np.float32).reshape(spec.n_experts, H).astype(np.float64)
            lg = rw @ xin
            if dl.f["router_b"] is not None:
                lg += dl.f["router_b"].download(np.float32)
            s = np.sort(lg)[::-1]
            if s[spec.top_k - 1] - s[spec.top_k] <= 1e-5 * np.abs(lg).max():
                ambiguous.append(li)
                continue
            ref = bv.download(np.float32).astype(np.float64)
            out = bf.download(np.float32).astype(np.float64)
            worst = max(worst, float(np.abs(out - ref).max() / max(np.abs(ref - x).max(), 1e-30)))
            compared += 1
        same = bool(np.array_equal(bf.download(np.float32), got))
    finally:
        ctx.set_option(M.OPT_DECODE_KERNEL, kernel_opt)
        bf.free(), bv.free()
    return {"token": t_last, "bit_identical_to_eager_per_layer_chain": same, "layers_compared": compared,
            "tie_ambiguous_layers": ambiguous, "max_rel_err_vs_valu": worst, "tolerance": 2e-3,
            "pass": bool(same and compared > 0 and worst <= 2e-3)}


MFMA_FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8 (the f8f6f4 MFMA with an fp8 B operand)
MFMA_INT8_PEAK_TOPS = 5000.0  # MI355X dense int8


def bench_batched(a, ctx, M, W, spec, config, T, K, Wm, cpu_on):
    """One step = one batched forward of T tokens through one layer (router, top-k, grouped
    gate/up + activation, grouped down, combine). C5: 512 tokens through the Zipf-skewed
    GPT-OSS-shape layer; with --batched T on another config: T tokens through its layer 0
    (Q4_K layers take the grouped int8-MFMA path). Returns the JSON line's object."""
    dl = W.DeviceLayer(ctx, spec)
    dl.layer.reserve(T)
    H, I = spec.hidden, spec.inter
    x = W.x_tokens(spec, T)
    dx, dy = ctx.to_device(x), ctx.zeros((T, H))
    ctx.sync()
    g = None
    if not a.no_graph:
        ctx.graph_begin()
        dl.layer.forward_batched(dx, T, dy)
        g = ctx.graph_end()
    run = (lambda: g.launch()) if g else (lambda: dl.layer.forward_batched(dx, T, dy))
    for _ in range(Wm):
        run()
    ctx.sync()
    ctx.timer_start()
    for _ in range(K):
        run()
    ms = ctx.timer_stop()
    tok_s = K * T / (ms / 1e3)
    y = dy.download(np.float32)
    assert np.all(np.isfinite(y)), "non-finite output"
    log(f"timed {K} steps of {T} tokens: {ms:.2f} ms -> {tok_s:.1f} tok/s")
    ctx.set_option(M.OPT_PROFILE, 1)
    ctx.profile_reset()
    P = 4
    for _ in range(P):
        dl.layer.forward_batched(dx, T, dy)
    ctx.sync()
    kern = {}
    for name in ("router_logits", "topk", "group", "split_x", "grouped_gateup", "split_h", "grouped_down",
                 "split_q4k", "grouped_q4k_gateup", "grouped_q4k_down", "grouped_q4k_shared_gateup",
                 "grouped_q4k_shared_down", "shared_gate", "combine", "gateup", "down", "shared_gateup"):
        n, tot = ctx.profile_read(name)
        if n:
            kern[name] = (n, tot)
    ctx.set_option(M.OPT_PROFILE, 0)
    log("kernels: " + ", ".join(f"{k}: n={v[0]} avg={v[1] / v[0] * 1e3:.2f}us" for k, v in kern.items()))
    dom = max(kern, key=lambda k: kern[k][1])
    avg_ms = kern[dom][1] / kern[dom][0]
    pairs = T * spec.top_k
    flops = {"grouped_gateup": 2.0 * pairs * 2 * I * H, "grouped_down": 2.0 * pairs * H * I,
             "grouped_q4k_gateup": 2.0 * pairs * 2 * I * H, "grouped_q4k_down": 2.0 * pairs * H * I}
    bytes_step = W.batched_bytes(spec, T)
    roof = None
    if dom in flops:
        ach = flops[dom] / (avg_ms * 1e-3) / 1e12
        q4 = dom.startswith("grouped_q4k")
        peak = MFMA_INT8_PEAK_TOPS if q4 else MFMA_FP8_PEAK_TFLOPS
        tr = measured_traffic(config) if config == 5 and T == W.CONFIG_TOKENS[5] else None
        traffic = int(tr["bytes_per_launch"]) if tr and tr.get("kernel") == dom else None
        roof = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 1), "peak": peak,
                "unit": "TOP/s" if q4 else "TFLOP/s", "frac": round(ach / peak, 4), "traffic": traffic,
                "traffic_source": "profiles/traffic.json (rocprofv3 --pmc)" if traffic else None,
                "flops_per_launch": flops[dom], "avg_launch_us": round(avg_ms * 1e3, 2),
                "note": ("GEMM ops of the layer; the 2-term int8 activation split issues 2x this MFMA work"
                         if q4 else "GEMM flops of the layer; the 3-term e4m3 activation split issues 3x this "
                                    "MFMA work")}
    cpu = None
    if cpu_on:
        import oracle  # test infrastructure; used here only as the timed CPU baseline

        host = dict(spec=spec)
        host.update(dl.download_quant())
        host.update(W.float_tensors(spec))
        L = oracle.layer_from_host(host)
        threads = a.cpu_threads or os.cpu_count() or 1
        L.forward(x[:1], n_threads=threads)
        t0 = time.perf_counter()
        ns = 0
        while ns < T and time.perf_counter() - t0 < 10.0:  # about 10 s of CPU work
            L.forward(x[ns:ns + 8], n_threads=threads)
            ns += 8
        dt = time.perf_counter() - t0
        cpu = {"value": round(ns / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
               "host": host_cpu(),
               "sample": f"oracle (C restatement of the reference CPU path, {threads} threads) on {ns} of the "
                         f"{T} tokens"}
    workload = W.CONFIG_NAMES[5] if config == 5 else f"{W.CONFIG_NAMES[config]}: layer 0, batched {T} tokens"
    out = {
        "metric": "expert-FFN batched/prefill tokens/s + MFMA utilisation, GPT-OSS-20B shape",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(ms / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4-weights/e4m3x3-act/f32-acc" if spec.mxfp4 else "q4_k-weights/int8x2-act/i32-f32-acc",
        "data": "synthetic (seeded SplitMix64 weights generated on the GPU; x ~ N(0,1)"
                + ("; Zipf(1.1) router skew)" if spec.zipf_s else ")"),
        "config": {"workload": workload, "config_id": config, "tokens": T, "hidden": H, "inter": I,
                   "experts": spec.n_experts, "top_k": spec.top_k, "graph": g is not None},
        "hbm_gbs": round(bytes_step * K / (ms / 1e3) / 1e9, 1),
        "hbm_frac": round(bytes_step * K / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_step": bytes_step,
        "roofline": roof, "cpu_baseline": cpu,
    }
    if g:
        g.close()
    dx.free(), dy.free()
    dl.close()
    return out


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration()
        return
    if a.probe:
        probes()
        return
    if a.probe_flags:
        probe_flags()
        return
    if a.probe_eager:
        probes_eager()
        return
    if a.trace:
        trace_decode(a)
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the MoE path is measured on "
                          "one MI355X; multi-GPU expert parallelism is a design note, not a run",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    import moe_rocm as M
    from moe_rocm import workloads as W

    ctx = M.Context(0)
    kernel_opt = {"auto": M.DECODE_AUTO, "valu": M.DECODE_VALU, "fused": M.DECODE_FUSED}[a.kernel]
    ctx.set_option(M.OPT_DECODE_KERNEL, kernel_opt)
    if a.config == 5 or a.batched:
        T = a.batched or W.CONFIG_TOKENS[5]
        K = a.steps if a.steps != 256 else 20
        out = bench_batched(a, ctx, M, W, W.config_layers(a.config)[0], a.config, T, K, a.warmup,
                            not a.no_cpu_baseline)
        print(json.dumps(out), flush=True)
        ctx.close()
        return
    out, ok = bench_decode(a, ctx, M, W, a.config, a.steps, a.warmup, kernel_opt, not a.no_cpu_baseline,
                           a.profile_tokens)
    headline = a.config == 2 and a.batched == 0 and a.decode == "layers" and not a.residual
    if headline and not a.no_extra_configs:
        out["extra_configs"] = extra_configs(a, ctx, M, W, kernel_opt)
    print(json.dumps(out), flush=True)
    ctx.close()
    if not ok:
        log("output check FAILED: the timed pipeline's outputs disagree with the eager VALU path")
        sys.exit(1)


# The other configurations, measured after the headline in the default run: decode tokens
# through every layer of C1 (8 independent layer copies), C3 and C4, and the C5 batched step,
# each with fewer timed steps and no CPU leg, so the whole default run stays within minutes.
# "2c": C2 with the hidden state carried through the layers by mr_moe_forward_residual (fused
# post-attention norm and residual add), the path a model's decode takes
EXTRA_STEPS = {1: 512, "2c": 256, 3: 256, 4: 256, 5: 20}


def extra_configs(a, ctx, M, W, kernel_opt) -> list:
    import copy

    rows = []
    for key, K in EXTRA_STEPS.items():
        t0 = time.perf_counter()
        cfg = 2 if key == "2c" else key
        if cfg == 5:
            o = bench_batched(a, ctx, M, W, W.config_layers(5)[0], 5, W.CONFIG_TOKENS[5], K, 3, False)
            ok = True
        else:
            ac = a
            if key == "2c":
                ac = copy.copy(a)
                ac.decode = "chain"
            o, ok = bench_decode(ac, ctx, M, W, cfg, K, 4, kernel_opt, False, 4)
        r = o["roofline"] or {}
        workload = o["config"]["workload"]
        if key == "2c":
            workload += "; fused post-attention RMSNorm + residual, hidden state carried through the layers"
        rows.append({"config_id": cfg, "workload": workload, "metric": o["metric"],
                     "value": o["value"], "unit": o["unit"], "steps": o["steps"], "ms_per_step": o["ms_per_step"],
                     "dtype": o["dtype"], "kernel": r.get("kernel"), "avg_launch_us": r.get("avg_launch_us"),
                     "roofline_bound": r.get("bound"), "achieved": r.get("achieved"), "peak": r.get("peak"),
                     "roofline_unit": r.get("unit"), "frac": r.get("frac"), "hbm_frac": o.get("hbm_frac"),
                     "output_check_pass": o["output_check"]["pass"] if "output_check" in o else None,
                     "seconds": round(time.perf_counter() - t0, 1)})
        if key == "2c":
            rows[-1]["decode"] = "chain"
        log(f"extra C{key}: {o['value']} {o['unit']}, frac {r.get('frac')}, {rows[-1]['seconds']} s")
        if not ok:
            log(f"output check FAILED on C{key}")
            sys.exit(1)
    return rows


def bench_decode(a, ctx, M, W, config, K, Wm, kernel_opt, cpu_on, profile_tokens):
    """Decode tokens through every layer of config `config` (K timed after Wm warmup tokens,
    one graph per token): the JSON line's object and whether the output check passed."""
    specs = W.config_layers(config)
    n_layers = len(specs)
    n_tok = K + Wm
    t0 = time.perf_counter()
    if a.decode == "layers":
        stack = W.DecodeStack(ctx, specs, residual=a.residual, prefetch_hint=not a.no_prefetch_hint)
    else:
        stack = W.ChainStack(ctx, specs, prefetch_hint=not a.no_prefetch_hint)
    layers = stack.layers
    log(f"built {n_layers} layers in {time.perf_counter() - t0:.1f}s")
    # inputs (x[token][layer], or h[token] for a carried hidden state) resident in HBM before
    # the timed region
    stack.load(stack.inputs(n_tok))
    if not a.no_graph:
        t0 = time.perf_counter()
        stack.capture()
        log(f"captured {len(stack.graphs)} token graphs in {time.perf_counter() - t0:.1f}s")

    for t in range(Wm):
        stack.run(t)
    ctx.sync()
    wall0 = time.perf_counter()
    ctx.timer_start()
    for t in range(Wm, n_tok):
        stack.run(t)
    ms = ctx.timer_stop()
    wall = time.perf_counter() - wall0
    ctx.sync()  # also reports a fused launch whose cross-workgroup wait ran out
    tok_s = K / (ms / 1e3)
    if config == 1:  # unit: one token through one layer (the 8 instances are independent copies)
        tok_s = K * n_layers / (ms / 1e3)
    y = stack.outputs()
    assert np.all(np.isfinite(y)), "non-finite output"
    log(f"timed {K} tokens: {ms:.2f} ms (event), {wall * 1e3:.2f} ms (wall) -> {tok_s:.1f} tok/s")
    if a.decode == "layers":
        check = output_check(ctx, M, W, stack, y, n_tok - 1, kernel_opt)
    else:
        check = chain_check(ctx, M, stack, n_tok - 1, kernel_opt)
    log(f"output check: {check}")

    bytes_per_token = sum(s.weight_bytes_per_token() for s in specs)
    flops_per_token = sum(s.flops_per_token() for s in specs)

    # live per-kernel timing (HIP events around each launch, eager, same stream)
    ctx.set_option(M.OPT_PROFILE, 1)
    ctx.profile_reset()
    P = min(profile_tokens, n_tok)
    for t in range(P):
        stack.enqueue_token(t)
    ctx.sync()
    kern = {}
    for name in ("fused_layer", "gateup", "down", "router_logits", "topk", "shared_gateup",
                 "rms_norm", "residual_add"):
        n, tot = ctx.profile_read(name)
        if n:
            kern[name] = (n, tot)
    ctx.set_option(M.OPT_PROFILE, 0)
    dom = max(kern, key=lambda k: kern[k][1])
    n_dom, tot_dom = kern[dom]
    if set(kern) == {dom}:
        # one kernel per layer: its average launch is the timed region's event
        # time over the launches in it (no per-launch event overhead)
        avg_ms, avg_how = ms / (K * n_layers), "timed-region events / launches"
    else:
        avg_ms, avg_how = tot_dom / n_dom, "per-launch events (eager profile pass)"
    s0 = specs[0]
    t = s0.ggml_type
    mb = lambda r, c: M.synth.matrix_bytes(t, r, c)  # noqa: E731
    if dom == "fused_layer":
        per_launch = sum(s.weight_bytes_per_token() for s in specs) / n_layers
    elif dom == "gateup":
        per_launch = s0.top_k * (2 * mb(s0.inter, s0.hidden) + (2 * s0.inter * 4 if s0.expert_bias else 0)) + s0.hidden * 4
    elif dom == "down":
        per_launch = s0.top_k * (mb(s0.hidden, s0.inter) + (s0.hidden * 4 if s0.expert_bias else 0)) + s0.hidden * 4
    else:
        per_launch = s0.n_experts * s0.hidden * 4
    achieved = per_launch / (avg_ms * 1e-3) / 1e9
    log("kernels: " + ", ".join(f"{k}: n={v[0]} avg={v[1] / v[0] * 1e3:.2f}us" for k, v in kern.items()))

    unit = "layer-tokens/s" if config == 1 else "tokens/s"
    tr = measured_traffic(config)
    traffic = None if tr is None or tr.get("kernel") != dom else int(tr["bytes_per_launch"])

    cpu = None
    if cpu_on:
        threads = a.cpu_threads or os.cpu_count() or 1
        t0 = time.perf_counter()
        tok_cpu, n_cpu, sec = cpu_baseline(layers, specs, threads)
        log(f"cpu baseline: {tok_cpu:.3f} tok/s ({n_cpu} tokens x {n_layers} layers, {sec:.1f}s of oracle time) "
            f"in {time.perf_counter() - t0:.1f}s")
        cpu = {"value": round(tok_cpu * n_layers if config == 1 else tok_cpu, 3), "unit": unit, "cores": threads,
               "host": host_cpu(), "kind": "port",
               "sample": f"oracle (C restatement of the reference CPU path; MXFP4 matvec rows and F32 GEMV rows "
                         f"split over {threads} threads, Q4_K dequant single-threaded as in the reference): the same "
                         f"{n_cpu} decode tokens through each of the {n_layers} layers, one layer resident on the host "
                         f"at a time, {sec:.1f} s of CPU work"}

    out = {
        "metric": "expert-FFN decode tokens/s + achieved HBM GB/s (% peak), GPT-OSS-20B shape",
        "value": round(tok_s, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(ms / K, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # what the kernels compute: MXFP4 weights on the scaled MFMA against the activation
        # split into 4 e4m3 terms per 32-element block; Q4_K weights on the int8 MFMA against
        # the activation split into 2 int8 terms per 16-element group (int32 sums, f32 scaling)
        "dtype": "mxfp4-weights/e4m3x4-act/f32-acc" if s0.mxfp4 else "q4_k-weights/int8x2-act/i32-f32-acc",
        "data": "synthetic (seeded SplitMix64 weights generated on the GPU; x ~ N(0,1))",
        "config": {"workload": W.CONFIG_NAMES[config], "config_id": config,
                   "layers": n_layers, "tokens": K, "hidden": s0.hidden, "inter": s0.inter,
                   "experts": [s.n_experts for s in specs][:1] if config != 4 else "256..512",
                   "top_k": s0.top_k, "graph": not a.no_graph, "kernel": a.kernel,
                   "next_layer_hint": not a.no_prefetch_hint,
                   "fused_norm_residual": a.residual or a.decode != "layers", "decode": a.decode},
        "hbm_gbs": round(K / (ms / 1e3) * bytes_per_token / 1e9, 1),
        "hbm_frac": round(K / (ms / 1e3) * bytes_per_token / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_token": bytes_per_token,
        "tflops": round(K / (ms / 1e3) * flops_per_token / 1e12, 3),
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": int(per_launch),
                     "avg_launch_us": round(avg_ms * 1e3, 3), "avg_launch_method": avg_how,
                     "traffic_source": None if traffic is None else "profiles/traffic.json (rocprofv3 --pmc)"},
        "cpu_baseline": cpu,
        "output_check": check,
    }
    stack.close()
    return out, bool(check["pass"])


if __name__ == "__main__":
    main()
