#!/usr/bin/env python3
"""HCT decode throughput on one MI355X: decoded weight output GB/s.

Workload: the weight set of a Llama-3-8B decoder layer -- q,o 4096x4096;
k,v 1024x4096; gate,up 14336x4096; down 4096x14336 (218,103,808 elements),
values N(0, 0.02), seeded -- stored as HCT-T: 64x64 tiles, top 30% of each
tile's DCT coefficients (k = 1228) as a bitmap + INT4 with f16 scales,
LZ4-compressed in blocks of 13 whole tiles (15,652 bytes: the reference
HctWriter's default block size, 16 KiB, rounded down to whole tiles;
crates/haagenti-hct/src/tensor.rs:74,536).  One step decodes
32 such layers back to back into bf16 tensors: per layer one batched LZ4
launch (compressed -> tile bytes) and one batched tile launch (dequant +
scatter + inverse DCT on MFMA -> bf16).  Inputs are resident in HBM before
timing starts.  Synthetic data: a few distinct layers are encoded on the host
and replicated into 32 separate device buffers.

Prints one JSON line (see the roofline / cpu_baseline fields).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decoded weight output GB/s on 1 MI355X + % of HBM peak; vs host-CPU ref"
HBM_PEAK_GBS = 8000.0
SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
          ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
RHO = 0.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def encode_layer(H, seed, k, tb, tiles_per_block):
    """Host producer: HCT-T tiles + LZ4 blocks for the 7 tensors of a layer."""
    rng = np.random.default_rng(seed)
    comp_parts, in_off, in_len, out_off, out_cap = [], [], [], [], []
    tensors = []          # (name, rows, cols, scratch_offset, tiles_len)
    pos = spos = 0
    comp = H.Lz4Compressor()
    for name, rows, cols in SHAPES:
        w = rng.normal(0.0, 0.02, (rows, cols)).astype(np.float32)
        tiles = H.hctt_encode(w, k)
        del w
        blk = tiles_per_block * tb
        for s in range(0, tiles.size, blk):
            chunk = tiles[s:s + blk]
            c = comp.compress(chunk.tobytes())
            comp_parts.append(c)
            in_off.append(pos)
            in_len.append(len(c))
            out_off.append(spos + s)
            out_cap.append(chunk.size)
            pos += len(c)
        tensors.append((name, rows, cols, spos, tiles.size, tiles if seed == 0 and name == "q" else None))
        spos += tiles.size
    blob = np.frombuffer(b"".join(comp_parts), np.uint8)
    return dict(blob=blob, in_off=np.array(in_off, np.uint64), in_len=np.array(in_len, np.uint32),
                out_off=np.array(out_off, np.uint64), out_cap=np.array(out_cap, np.uint32),
                tensors=tensors, scratch_bytes=spos)


def cpu_baseline(O, layer, k, budget_s):
    """Oracle (C restatement of the reference CPU decode) on the host cores:
    LZ4 blocks -> tile bytes -> dequant + scatter + f32 IDCT, all threads."""
    nthreads = os.cpu_count() or 1
    n_elem = sum(r * c for _, r, c in SHAPES)
    reps, t_total = 0, 0.0
    while True:
        t0 = time.perf_counter()
        scratch, kinds, _ = O.lz4_decompress_batch(layer["blob"], layer["in_off"], layer["in_len"],
                                                   layer["out_off"], layer["out_cap"],
                                                   layer["scratch_bytes"], nthreads=nthreads)
        assert (kinds == 0).all()
        for name, rows, cols, soff, tlen, _ in layer["tensors"]:
            rc, _ = O.hctt_decode_tensor(scratch[soff:soff + tlen], rows, cols, k, nthreads=nthreads)
            assert rc == O.OK
        t_total += time.perf_counter() - t0
        reps += 1
        if t_total >= budget_s or reps >= 20:
            break
    gbs = reps * n_elem * 2 / t_total / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
            "sample": f"{reps} full Llama-3-8B layer decode(s) ({n_elem} elements each: LZ4 + "
                      f"dequant + scatter + f32 Makhoul IDCT), {nthreads} threads, output counted "
                      f"as bf16 bytes (2 B/element) like the GPU line; {t_total:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--distinct", type=int, default=2, help="distinct encoded layers")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--lz4-block", type=int, default=16384,
                    help="LZ4 block size in bytes before rounding down to whole tiles "
                         "(the reference HctWriter default is 16 KiB)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build "
              "decodes on a single MI355X; see DESIGN.md for how the path would shard).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import haagenti_amd as H

    torch.cuda.set_device(0)
    k = H.hctt_retain_count(RHO)
    tb = H.hctt_tile_bytes(k)
    tiles_per_block = max(1, args.lz4_block // tb)
    n_elem = sum(r * c for _, r, c in SHAPES)
    out_bytes_layer = n_elem * 2

    t0 = time.time()
    layers_host = [encode_layer(H, d, k, tb, tiles_per_block) for d in range(args.distinct)]
    log(f"encoded {args.distinct} distinct layer(s) in {time.time() - t0:.1f}s: "
        f"{layers_host[0]['blob'].size / 1e6:.1f} MB compressed, "
        f"{layers_host[0]['scratch_bytes'] / 1e6:.1f} MB tile bytes per layer")

    ctx = H.HipContext(0)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def u64(a):
        return torch.from_numpy(a.view(np.int64)).cuda()

    def u32(a):
        return torch.from_numpy(a.view(np.int32)).cuda()

    dev_tables = []
    for L in layers_host:
        dev_tables.append(dict(in_off=u64(L["in_off"]), in_len=u32(L["in_len"]),
                               out_off=u64(L["out_off"]), out_cap=u32(L["out_cap"]),
                               n=L["in_off"].size))
    d_comp, outs = [], []
    for l in range(args.layers):
        L = layers_host[l % args.distinct]
        d_comp.append(torch.from_numpy(L["blob"]).cuda())
        outs.append([torch.empty(r * c, dtype=torch.bfloat16, device="cuda") for _, r, c in SHAPES])
    scratch = [torch.empty(layers_host[0]["scratch_bytes"], dtype=torch.uint8, device="cuda")
               for _ in range(2)]
    status = torch.zeros(max(t["n"] for t in dev_tables) * 32, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    nlaunch = [0]
    ev = []

    def run_layer(l, timed):
        L = layers_host[l % args.distinct]
        T = dev_tables[l % args.distinct]
        s = scratch[l % 2]
        if timed:
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record(stream)
        rc = ctx.lz4_decompress_batch(d_comp[l], d_comp[l].numel(), T["in_off"], T["in_len"], s,
                                      T["out_off"], T["out_cap"], T["n"], status, stream=sp)
        assert rc == H.OK
        if timed:
            e1.record(stream)
        ctx.hctt_decode_batch([(s.data_ptr() + soff, tlen, rows, cols, k, outs[l][i])
                               for i, (name, rows, cols, soff, tlen, _) in enumerate(L["tensors"])],
                              dtype=H.BF16, stream=sp)
        if timed:
            e2.record(stream)
            ev.append((e0, e1, e2))

    def step(timed=False):
        for l in range(args.layers):
            run_layer(l, timed)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # correctness spot check of layer 0 / q against the oracle
    codes = status.cpu().numpy().view(np.int32)[0::8][:dev_tables[-1]["n"]]
    assert (codes == 0).all(), "LZ4 block errors"
    check = None
    try:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        name, rows, cols, soff, tlen, qtiles = layers_host[0]["tensors"][0]
        sub_rows = 256
        rc, ref = O.hctt_decode_tensor(qtiles[: (sub_rows // 64) * (cols // 64) * tb], sub_rows, cols, k)
        got = outs[0][0].view(rows, cols)[:sub_rows].float().cpu().numpy()
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        check = float(np.abs(got - ref).max() / rms)
        log(f"spot check layer0/q rows 0..{sub_rows}: max|bf16 - oracle f32| = {check:.2e} x RMS")
    except Exception as ex:  # oracle library missing is not fatal for timing
        O = None
        log(f"spot check skipped: {ex}")

    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    ev.clear()
    t_start.record(stream)
    w0 = time.perf_counter()
    for _ in range(args.steps):
        step(timed=True)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    total_ms = t_start.elapsed_time(t_end)
    ms_step = total_ms / args.steps
    value = out_bytes_layer * args.layers / (ms_step / 1e3) / 1e9

    lz4_ms = [a.elapsed_time(b) for a, b, _ in ev]
    tile_ms = [b.elapsed_time(c) for _, b, c in ev]
    in_tile_bytes = layers_host[0]["scratch_bytes"]
    comp_bytes = layers_host[0]["blob"].size
    tile_avg = float(np.mean(tile_ms))
    lz4_avg = float(np.mean(lz4_ms))
    tile_gbs = (in_tile_bytes + out_bytes_layer) / (tile_avg / 1e3) / 1e9
    lz4_gbs = (comp_bytes + in_tile_bytes) / (lz4_avg / 1e3) / 1e9
    log(f"per layer: lz4 {lz4_avg * 1e3:.1f} us ({lz4_gbs:.0f} GB/s in+out), "
        f"tiles {tile_avg * 1e3:.1f} us ({tile_gbs:.0f} GB/s in+out, "
        f"{256 * n_elem / (tile_avg / 1e3) / 1e12:.0f} TFLOP/s algorithmic); wall {wall:.3f}s")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16-split-mfma/f32",
        "data": "synthetic (N(0,0.02) weights, seeded; %d distinct layers replicated)" % args.distinct,
        "config": {"workload": "llama3-8b-layer-hct-decode", "layers": args.layers,
                   "elements_per_layer": n_elem, "rho": RHO, "k": k, "tile": 64,
                   "tile_bytes": tb, "lz4_block_tiles": tiles_per_block, "out_dtype": "bf16",
                   "hct_bytes_per_layer": in_tile_bytes, "lz4_bytes_per_layer": comp_bytes},
        "roofline": {"bound": "hbm", "achieved": round(tile_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(tile_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "hctt_decode_kernel<bf16>",
                     "avg_launch_us": round(tile_avg * 1e3, 2)},
        "kernels_us": {"lz4_batch_kernel": round(lz4_avg * 1e3, 2),
                       "hctt_decode_kernel": round(tile_avg * 1e3, 2)},
        "spot_check_max_err_over_rms": check,
    }
    if not args.no_cpu and O is not None:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(O, layers_host[0], k, args.cpu_budget)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
