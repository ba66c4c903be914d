#!/usr/bin/env python3
"""HCT decode throughput on one MI355X: decoded weight output GB/s.

Default workload (--workload llama3-8b-layer): the weight set of a
Llama-3-8B decoder layer -- q,o 4096x4096; k,v 1024x4096; gate,up
14336x4096; down 4096x14336 (218,103,808 elements), values N(0, 0.02),
seeded -- stored as HCT-T: 64x64 tiles, top 30% of each tile's DCT
coefficients (k = 1228) as a bitmap + INT4 with f16 scales, LZ4-compressed
in blocks of 13 whole tiles (15,652 bytes: the reference HctWriter's default
block size, 16 KiB, rounded down to whole tiles;
crates/haagenti-hct/src/tensor.rs:74,536).  One step decodes 32 such layers
back to back into bf16 tensors: per four layers (--layers-per-launch) one
hh_hctt_decode_lz4_fused call, i.e. one launch that decodes the layers' LZ4
blocks into LDS and their tiles (dequant + scatter + inverse DCT on MFMA) to
bf16 (four layers share a launch's start-up, pipeline fill and drain).
Inputs are resident in HBM before timing starts.  The step time brackets all
32 layers, with nothing recorded between the launches; the roofline's average
launch is the step time over the launches (launch gaps included, so it
cannot exceed a launch's share of the step).  --path two-launch decodes each layer with
hh_hctt_decode_lz4_batch (an LZ4 launch into a scratch buffer, then the tile
launch); its per-kernel times come from HIP events around the launches of
every 8th layer of the timed steps (--kernel-sample).

Other workloads (one JSON line each, same contract):
  int4-4096        4096x4096 f32 N(0, 0.02) through quantize_int4 (block 32,
                   truncated f16 scales); GPU dequant to f32, bit-exact mode
  lz4-256mib       4096 independent 64 KiB blocks (256 MiB out), each packed
                   INT4 nibbles of N(0, 0.02) weights or the same with half of
                   the 256-byte spans zeroed, seeded coin per block
  idct-8192        one 8192x8192 tensor as HCT-T at 25% retention (k = 1024),
                   dequant + scatter + tile inverse DCT to bf16
  llama70b-stream  80 Llama-70B-shaped layers (q,o 8192^2; k,v 1024x8192;
                   gate,up,down 28672x8192 / 8192x28672), per-tensor retention
                   U[0.10, 0.50]; compressed layers in pinned host memory,
                   H2D copies on a copy stream overlapped with decode into a
                   double-buffered bf16 layer slot; --from-file reads every
                   layer from its seven HCT v2 files (mmap) into double-
                   buffered pinned staging instead
  xxh3-256mib      HCT v2 block validation: XXH3-64 of the 4096 compressed
                   blocks of lz4-256mib (one wavefront per block), the
                   checksum HctReaderV2 verifies per block; value = hashed
                   bytes per second (the kernel reads its input once)
  hct3-4096        one 4096x4096 N(0, 0.02) tensor (--hct3-size n: n x n)
                   as an HCT V3 fragment container (whole-tensor DCT, turbo
                   defaults: top 20 %, f16 coefficients); GPU bitmap scatter
                   + whole-matrix inverse DCT, bf16 out: by default the FFT
                   route (row transforms through an f32 FFT in LDS and two
                   transposes; roofline against HBM), --dct-route dense the
                   two hand-written split-f16 MFMA products (five f16 passes,
                   f32 accumulation; roofline against the f16 MFMA peak)
  hbm-copy         a 1 GiB device copy by the library's streaming copy kernel
                   (hh_hbm_copy): the HBM reference rate and the calibration
                   for the FETCH_SIZE / WRITE_SIZE counters

Synthetic data throughout (no network): a few distinct encodings are made on
the host and replicated or cycled.  `roofline.traffic` is read from
profiles/traffic.json (HBM bytes per launch of the dominant kernel, from
rocprofv3 FETCH_SIZE and WRITE_SIZE runs scaled by the copy calibration) when
that file holds the workload, else null.
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
L8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
       ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
L70B = [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
        ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672)]
RHO_8B = 0.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads():
    return os.cpu_count() or 1


def oracle():
    """The CPU oracle (test infrastructure) used only for the cpu_baseline leg
    and the spot check; None when its library is not built."""
    try:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        O.lib()
        return O
    except Exception as ex:  # the GPU timing does not depend on it
        log(f"oracle unavailable: {ex}")
        return None


def traffic_for(workload):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f).get(workload)
        return None if t is None else t["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def fused_traffic(lpl):
    """Traffic of a fused launch over `lpl` layers: measured for that many layers when
    profiles/traffic.json holds it, else the one-layer measurement scaled by `lpl`."""
    key = f"llama3-8b-layer:fused-x{lpl}"
    if lpl > 1 and traffic_for(key) is not None:
        return {"traffic_key": key}
    return {"traffic_key": "llama3-8b-layer:fused", "traffic_scale": lpl}


def roofline(workload, kernel, algo_bytes, avg_s, extra=None, traffic_key=None, traffic_scale=1):
    achieved = algo_bytes / avg_s / 1e9
    traffic = traffic_for(traffic_key or workload)  # measured per launch of one unit (e.g. one layer)
    r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None if traffic is None else traffic * traffic_scale,
         "kernel": kernel, "avg_launch_us": round(avg_s * 1e6, 2),
         "algorithmic_bytes_per_launch": int(algo_bytes)}
    if extra:
        r.update(extra)
    return r


def line(workload, value, ms_step, args, dtype, data, config, roof, cpu, extra=None):
    d = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
         "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
         "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
         "data": data, "config": dict(workload=workload, **config), "roofline": roof,
         "cpu_baseline": cpu}
    if extra:
        d.update(extra)
    return d


class Timed:
    """HIP events on one stream around a region (torch.cuda.Event records on
    the stream it is given, which is the stream the kernels are launched on)."""

    def __init__(self, torch, stream, reserve=0):
        self.torch, self.stream = torch, stream
        self.pairs = []
        # HIP creates an event's signal at its first record, and growing the
        # runtime's signal pool can stall the host for milliseconds while the
        # GPU runs dry: events used inside a timed loop are created and
        # recorded once beforehand
        self.free = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reserve)]
        for e in self.free:
            e.record(stream)
        if reserve:
            torch.cuda.synchronize()

    def _event(self):
        return self.free.pop() if self.free else self.torch.cuda.Event(enable_timing=True)

    def start(self):
        e = self._event()
        e.record(self.stream)
        return e

    def stop(self, e0):
        e1 = self._event()
        e1.record(self.stream)
        self.pairs.append((e0, e1))

    def mean_s(self):
        return float(np.mean([a.elapsed_time(b) for a, b in self.pairs])) / 1e3

    def spread(self):
        """(min, median, max) launch time in microseconds."""
        t = np.array([a.elapsed_time(b) for a, b in self.pairs]) * 1e3
        return float(t.min()), float(np.median(t)), float(t.max())


LZ4_KERNEL_NAMES = {"auto": "lz4_ring_kernel<4096, 4096>", "seq": "lz4_seq_kernel<4096, 4096>", "seq8": "lz4_seq_kernel<8192, 2048>",
                    "ring4": "lz4_ring_kernel<4096, 4096>", "ring8": "lz4_ring_kernel<8192, 2048>",
                    "ring16": "lz4_ring_kernel<16384, 3072>", "ring32": "lz4_ring_kernel<32768, 4096>",
                    "window": "lz4_batch_kernel"}


def new_ctx(H, args):
    ctx = H.HipContext(0)
    ctx.set_lz4_decoder(args.lz4_decoder)
    ctx.set_dct_route(args.dct_route)
    ctx.set_pipeline_route(args.pipeline_route)
    return ctx


def warm(step, args):
    """Untimed steps right before the timed region: the checks before it
    leave the GPU idle and its clocks fall back."""
    import torch
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()


def devtab(torch, a):
    a = np.ascontiguousarray(a)
    view = np.int64 if a.dtype == np.uint64 else np.int32
    return torch.from_numpy(a.view(view).copy()).cuda()


# ---------------------------------------------------------------- producers
def encode_tensor_lz4(H, w, k, tiles_per_block):
    """HCT-T tiles of w, cut into LZ4 blocks of whole tiles (host producer)."""
    tb = H.hctt_tile_bytes(k)
    tiles = H.hctt_encode(w, k)
    comp = H.Lz4Compressor()
    blk = tiles_per_block * tb
    parts, lens, outs, caps = [], [], [], []
    for s in range(0, tiles.size, blk):
        chunk = tiles[s:s + blk]
        c = comp.compress(chunk.tobytes())
        parts.append(c)
        lens.append(len(c))
        outs.append(s)
        caps.append(chunk.size)
    return tiles, parts, lens, outs, caps


def encode_layer(H, shapes, ks, seed, block_bytes, keep_first=False):
    """One layer: for each tensor its HCT-T tiles LZ4-compressed in blocks of
    whole tiles; block tables index one concatenated blob and one scratch."""
    rng = np.random.default_rng(seed)
    parts, in_off, in_len, out_off, out_cap, tensors = [], [], [], [], [], []
    pos = spos = 0
    for (name, rows, cols), k in zip(shapes, ks):
        w = rng.normal(0.0, 0.02, (rows, cols)).astype(np.float32)
        tb = H.hctt_tile_bytes(k)
        tiles, p, lens, outs, caps = encode_tensor_lz4(H, w, k, max(1, block_bytes // tb))
        del w
        for c, ln, o, cp in zip(p, lens, outs, caps):
            parts.append(c)
            in_off.append(pos)
            in_len.append(ln)
            out_off.append(spos + o)
            out_cap.append(cp)
            pos += ln
        tensors.append(dict(name=name, rows=rows, cols=cols, k=k, soff=spos, tlen=tiles.size,
                            tiles=tiles if keep_first and not tensors else None))
        spos += tiles.size
    return dict(blob=np.frombuffer(b"".join(parts), np.uint8), in_off=np.array(in_off, np.uint64),
                in_len=np.array(in_len, np.uint32), out_off=np.array(out_off, np.uint64),
                out_cap=np.array(out_cap, np.uint32), tensors=tensors, scratch_bytes=spos)


def cpu_layer_decode(O, layer, reps_budget_s, max_reps=1000, tensor_subset=None):
    """Oracle decode (LZ4 blocks -> tile bytes -> dequant + scatter + f32
    Makhoul IDCT) on all host threads; returns (reps, seconds, elements)."""
    nthreads = cpu_threads()
    reps, t_total, n_elem = 0, 0.0, 0
    tens = layer["tensors"] if tensor_subset is None else [layer["tensors"][i] for i in tensor_subset]
    while True:
        t0 = time.perf_counter()
        scratch, kinds, _ = O.lz4_decompress_batch(layer["blob"], layer["in_off"], layer["in_len"],
                                                   layer["out_off"], layer["out_cap"],
                                                   layer["scratch_bytes"], nthreads=nthreads)
        assert (kinds == 0).all()
        n_elem = 0
        for T in tens:
            rc, _ = O.hctt_decode_tensor(scratch[T["soff"]:T["soff"] + T["tlen"]], T["rows"],
                                         T["cols"], T["k"], nthreads=nthreads)
            assert rc == O.OK
            n_elem += T["rows"] * T["cols"]
        t_total += time.perf_counter() - t0
        reps += 1
        if t_total >= reps_budget_s or reps >= max_reps:
            return reps, t_total, n_elem


# ---------------------------------------------------------------- workloads
def wl_llama3_8b_layer(args, torch, H, O):
    k = H.hctt_retain_count(RHO_8B)
    tb = H.hctt_tile_bytes(k)
    tiles_per_block = max(1, args.lz4_block // tb)
    n_elem = sum(r * c for _, r, c in L8B)
    out_bytes_layer = n_elem * 2

    t0 = time.time()
    layers_host = [encode_layer(H, L8B, [k] * len(L8B), d, tiles_per_block * tb, keep_first=d == 0)
                   for d in range(args.distinct)]
    log(f"encoded {args.distinct} distinct layer(s) in {time.time() - t0:.1f}s: "
        f"{layers_host[0]['blob'].size / 1e6:.1f} MB compressed, "
        f"{layers_host[0]['scratch_bytes'] / 1e6:.1f} MB tile bytes per layer")

    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    tabs = [dict(in_off=devtab(torch, L["in_off"]), in_len=devtab(torch, L["in_len"]),
                 out_off=devtab(torch, L["out_off"]), out_cap=devtab(torch, L["out_cap"]),
                 n=L["in_off"].size) for L in layers_host]
    fused = args.path == "fused"
    # fused path: layers_per_launch consecutive layers per launch (their
    # compressed blocks in one device buffer, the block offsets shifted)
    lpl = args.layers_per_launch if fused else 1
    groups = [list(range(g, min(g + lpl, args.layers))) for g in range(0, args.layers, lpl)]
    d_comp, outs, gdata = [], [], []
    for l in range(args.layers):
        outs.append([torch.empty(r * c, dtype=torch.bfloat16, device="cuda") for _, r, c in L8B])
    if lpl == 1:
        for l in range(args.layers):
            d_comp.append(torch.from_numpy(layers_host[l % args.distinct]["blob"].copy()).cuda())
    else:
        for grp in groups:
            Ls = [layers_host[l % args.distinct] for l in grp]
            base = np.cumsum([0] + [L["blob"].size for L in Ls[:-1]]).astype(np.uint64)
            gdata.append(dict(
                d=torch.from_numpy(np.concatenate([L["blob"] for L in Ls])).cuda(),
                in_off=devtab(torch, np.concatenate([L["in_off"] + b for L, b in zip(Ls, base)])),
                in_len=devtab(torch, np.concatenate([L["in_len"] for L in Ls])),
                n=sum(int(L["in_off"].size) for L in Ls),
                desc=[(t["rows"], t["cols"], k, outs[l][i]) for l, L in zip(grp, Ls)
                      for i, t in enumerate(L["tensors"])]))
    scratch = [torch.empty(layers_host[0]["scratch_bytes"], dtype=torch.uint8, device="cuda")
               for _ in range(2)]
    status = torch.zeros(max([t["n"] for t in tabs] + [g["n"] for g in gdata]) * 32, dtype=torch.uint8,
                         device="cuda")
    torch.cuda.synchronize()
    # per-kernel HIP events bracket the launches of every kernel_sample-th
    # layer of the timed steps (an event record between two launches costs
    # the stream a few microseconds)
    sampled = [l for l in range(args.layers) if l % args.kernel_sample == 0]
    t_lz4, t_tile = (Timed(torch, stream, args.steps * len(sampled)),
                     Timed(torch, stream, args.steps * len(sampled)))

    def run_group(gi):
        # layers_per_launch layers in one fused launch
        G = gdata[gi]
        rc = ctx.hctt_decode_lz4_fused(G["d"], G["d"].numel(), G["in_off"], G["in_len"], G["n"], status,
                                       G["desc"], tiles_per_block, dtype=H.BF16, stream=sp)
        assert rc == H.OK

    def run_layer(l, timed):
        L = layers_host[l % args.distinct]
        T = tabs[l % args.distinct]
        if fused:
            # the layer in one launch: LZ4 blocks -> tile bytes in LDS -> bf16
            # (no events between the launches: the step time / layers is the
            # launch time)
            fdesc = [(t["rows"], t["cols"], k, outs[l][i]) for i, t in enumerate(L["tensors"])]
            rc = ctx.hctt_decode_lz4_fused(d_comp[l], d_comp[l].numel(), T["in_off"], T["in_len"], T["n"], status,
                                           fdesc, tiles_per_block, dtype=H.BF16, stream=sp)
            assert rc == H.OK
            return
        s = scratch[l % 2]
        desc = [(s.data_ptr() + t["soff"], t["tlen"], t["rows"], t["cols"], k, outs[l][i])
                for i, t in enumerate(L["tensors"])]
        if not (timed and l % args.kernel_sample == 0):
            # the layer in one call: LZ4 blocks -> scratch -> bf16 tensors
            ctx.hctt_decode_lz4_batch(d_comp[l], d_comp[l].numel(), T["in_off"], T["in_len"], s, T["out_off"],
                                      T["out_cap"], T["n"], status, desc, dtype=H.BF16, stream=sp)
            return
        # sampled layers: the same two launches, with events between them
        e = t_lz4.start()
        rc = ctx.lz4_decompress_batch(d_comp[l], d_comp[l].numel(), T["in_off"], T["in_len"], s,
                                      T["out_off"], T["out_cap"], T["n"], status, stream=sp)
        assert rc == H.OK
        t_lz4.stop(e)
        e = t_tile.start()
        ctx.hctt_decode_batch(desc, dtype=H.BF16, stream=sp)
        t_tile.stop(e)

    def step(timed=False):
        if lpl > 1:
            for gi in range(len(groups)):
                run_group(gi)
            return
        for l in range(args.layers):
            run_layer(l, timed)

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    codes = status.cpu().numpy().view(np.int32)[0::8][:(gdata[-1]["n"] if gdata else tabs[-1]["n"])]
    assert (codes == 0).all(), "LZ4 block errors"
    check = None
    if O is not None:
        T0 = layers_host[0]["tensors"][0]
        sub = 256
        rc, ref = O.hctt_decode_tensor(T0["tiles"][: (sub // 64) * (T0["cols"] // 64) * tb], sub,
                                       T0["cols"], k)
        got = outs[0][0].view(T0["rows"], T0["cols"])[:sub].float().cpu().numpy()
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        check = float(np.abs(got - ref).max() / rms)
        log(f"spot check layer0/q rows 0..{sub}: max|bf16 - oracle f32| = {check:.2e} x RMS")

    warm(step, args)
    ta, tz = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ta.record(stream)
    for _ in range(args.steps):
        step(timed=True)
    tz.record(stream)
    torch.cuda.synchronize()
    ms_step = ta.elapsed_time(tz) / args.steps
    value = out_bytes_layer * args.layers / (ms_step / 1e3) / 1e9
    in_tile = layers_host[0]["scratch_bytes"]
    comp_bytes = layers_host[0]["blob"].size
    tile_s = ms_step / 1e3 / args.layers if fused else t_tile.mean_s()
    lz4_s = t_lz4.mean_s() if not fused else None
    if fused:
        log(f"per layer: fused LZ4 + tiles {tile_s * 1e6:.1f} us ({(comp_bytes + out_bytes_layer) / tile_s / 1e9:.0f} "
            f"GB/s compressed in + bf16 out; the {in_tile / 1e6:.1f} MB of tile bytes stay in LDS)")
    else:
        log(f"per layer: lz4 {lz4_s * 1e6:.1f} us ({(comp_bytes + in_tile) / lz4_s / 1e9:.0f} GB/s "
            f"in+out), tiles {tile_s * 1e6:.1f} us ({(in_tile + out_bytes_layer) / tile_s / 1e9:.0f} "
            f"GB/s in+out)")
        log("tile launch us min/median/max %.1f / %.1f / %.1f; sampled tile time per step (ms): %s" % (
            *t_tile.spread(), " ".join("%.2f" % (sum(a.elapsed_time(b) for a, b in
                                                      t_tile.pairs[i * len(sampled):(i + 1) * len(sampled)]))
                                       for i in range(args.steps))))
    cpu = None
    if not args.no_cpu and O is not None:
        log("cpu baseline ...")
        reps, secs, ne = cpu_layer_decode(O, layers_host[0], args.cpu_budget)
        cpu = {"value": round(reps * ne * 2 / secs / 1e9, 3), "unit": "GB/s", "cores": cpu_threads(),
               "kind": "port",
               "sample": f"{reps} full Llama-3-8B layer decode(s) ({ne} elements each: LZ4 + dequant "
                         f"+ scatter + f32 Makhoul IDCT), {cpu_threads()} threads, output counted as "
                         f"bf16 bytes like the GPU line; {secs:.1f} s"}
    return line("llama3-8b-layer", value, ms_step, args, "f16-split-mfma/f32",
                f"synthetic (N(0,0.02) weights, seeded; {args.distinct} distinct layers replicated)",
                {"layers": args.layers, "layers_per_launch": lpl, "elements_per_layer": n_elem, "rho": RHO_8B, "k": k,
                 "tile": 64, "tile_bytes": tb, "lz4_block_tiles": tiles_per_block,
                 "out_dtype": "bf16", "hct_bytes_per_layer": in_tile,
                 "lz4_bytes_per_layer": comp_bytes},
                (roofline("llama3-8b-layer:fused", "hctt_lz4_fused_kernel<bf16>",
                          lpl * (comp_bytes + out_bytes_layer), lpl * tile_s,
                          **fused_traffic(lpl)) if fused else
                 roofline("llama3-8b-layer", "hctt_decode_kernel<bf16>", in_tile + out_bytes_layer, tile_s)),
                cpu,
                ({"path": "fused", "kernels_us": {"hctt_lz4_fused_kernel": round(lpl * tile_s * 1e6, 2)},
                  "per_layer_us": round(tile_s * 1e6, 2),
                  "avg_launch_is": "step time / launches (back-to-back launches of layers_per_launch layers, "
                                   "no events between them)",
                  "spot_check_max_err_over_rms": check} if fused else
                 {"path": "two-launch",
                  "kernels_us": {"lz4_kernel": round(lz4_s * 1e6, 2),
                                 "hctt_decode_kernel": round(tile_s * 1e6, 2)},
                  "lz4_roofline": {"achieved": round((comp_bytes + in_tile) / lz4_s / 1e9, 1),
                                   "frac": round((comp_bytes + in_tile) / lz4_s / 1e9 / HBM_PEAK_GBS, 4)},
                  "spot_check_max_err_over_rms": check}))


def wl_int4(args, torch, H, O):
    n = 4096 * 4096
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, n).astype(np.float32)
    q = H.quantize_int4(w)
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    dq = torch.from_numpy(q.copy()).cuda()
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    launches = 200

    def step():
        for _ in range(launches):
            ctx.dequant_int4(dq, q.size, n, out, dtype=H.F32, stream=sp)

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    exact = None
    if O is not None:
        ref = O.dequantize_int4(q, n, threads=cpu_threads())
        exact = bool((out.cpu().numpy().view(np.uint32) == ref.view(np.uint32)).all())
        log(f"bit-exact vs oracle: {exact}")
    warm(step, args)
    T = Timed(torch, stream)
    e = T.start()
    for _ in range(args.steps):
        step()
    T.stop(e)
    torch.cuda.synchronize()
    ms_step = T.mean_s() * 1e3 / args.steps
    per = ms_step / 1e3 / launches
    out_b = n * 4
    algo = q.size + out_b
    cpu = None
    if not args.no_cpu and O is not None:
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_budget:
            O.dequantize_int4(q, n, threads=cpu_threads())
            reps += 1
        secs = time.perf_counter() - t0
        cpu = {"value": round(reps * out_b / secs / 1e9, 3), "unit": "GB/s", "cores": cpu_threads(),
               "kind": "port", "sample": f"{reps} dequantizations of the full 4096x4096 tensor to "
                                         f"f32, {cpu_threads()} threads, {secs:.1f} s"}
    return line("int4-4096", out_b / per / 1e9, ms_step, args, "f32",
                "synthetic (4096x4096 N(0,0.02), seed 1)",
                {"elements": n, "group": 32, "in_bytes": int(q.size), "out_dtype": "f32",
                 "launches_per_step": launches},
                roofline("int4-4096", "dequant_int4_kernel<f32>", algo, per), cpu,
                {"bit_exact": exact})


def config2_blocks(H, seed=3, nsrc=64, nblocks=4096):
    rng = np.random.default_rng(seed)
    srcs = []
    for i in range(nsrc):
        w = rng.normal(0, 0.02, 131072).astype(np.float32)
        nib = H.quantize_int4(w)[2 * 4096:].copy()
        if i % 2:
            nib[np.repeat(rng.random(256) < 0.5, 256)] = 0
        srcs.append(nib.tobytes())
    comp = [H.Lz4Compressor().compress(s) for s in srcs]
    pick = rng.integers(0, nsrc, nblocks)
    in_len = np.array([len(comp[i]) for i in pick], np.uint32)
    in_off = np.concatenate([[0], np.cumsum(in_len.astype(np.uint64))[:-1]]).astype(np.uint64)
    blob = np.frombuffer(b"".join(comp[i] for i in pick), np.uint8)
    return srcs, pick, blob, in_off, in_len


def wl_lz4(args, torch, H, O):
    nb = 4096
    srcs, pick, blob, in_off, in_len = config2_blocks(H)
    out_off = np.arange(nb, dtype=np.uint64) * 65536
    out_cap = np.full(nb, 65536, np.uint32)
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    d_in = torch.from_numpy(blob.copy()).cuda()
    d_out = torch.empty(nb * 65536, dtype=torch.uint8, device="cuda")
    st = torch.zeros(nb * 32, dtype=torch.uint8, device="cuda")
    a = (d_in, d_in.numel(), devtab(torch, in_off), devtab(torch, in_len), d_out,
         devtab(torch, out_off), devtab(torch, out_cap), nb, st)
    launches = 10

    def step():
        for _ in range(launches):
            assert ctx.lz4_decompress_batch(*a, stream=sp) == H.OK

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    codes = st.cpu().numpy().view(np.int32)[0::8]
    assert (codes == 0).all()
    o = d_out.cpu().numpy()
    exact = all(o[j * 65536:(j + 1) * 65536].tobytes() == srcs[pick[j]] for j in range(nb))
    log(f"all {nb} blocks bit-exact: {exact}")
    warm(step, args)
    T = Timed(torch, stream)
    e = T.start()
    for _ in range(args.steps):
        step()
    T.stop(e)
    torch.cuda.synchronize()
    ms_step = T.mean_s() * 1e3 / args.steps
    per = ms_step / 1e3 / launches
    out_b = nb * 65536
    cpu = None
    if not args.no_cpu and O is not None:
        m = 1024
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_budget:
            O.lz4_decompress_batch(blob, in_off[:m], in_len[:m], out_off[:m], out_cap[:m],
                                   m * 65536, nthreads=cpu_threads())
            reps += 1
        secs = time.perf_counter() - t0
        cpu = {"value": round(reps * m * 65536 / secs / 1e9, 3), "unit": "GB/s",
               "cores": cpu_threads(), "kind": "port",
               "sample": f"{reps} x the first {m} of the 4096 blocks (64 MiB out each), "
                         f"{cpu_threads()} threads, {secs:.1f} s"}
    return line("lz4-256mib", out_b / per / 1e9, ms_step, args, "u8",
                "synthetic (64 distinct seeded blocks, seeded coin per block)",
                {"blocks": nb, "block_bytes": 65536, "in_bytes": int(blob.size),
                 "launches_per_step": launches},
                roofline("lz4-256mib", LZ4_KERNEL_NAMES[args.lz4_decoder], blob.size + out_b, per,
                         traffic_key={"auto": "lz4-256mib", "ring4": "lz4-256mib",
                                      "seq": "lz4-256mib:seq"}.get(args.lz4_decoder, "-")), cpu,
                {"bit_exact": exact})


def wl_idct(args, torch, H, O):
    rows = cols = 8192
    k = H.hctt_retain_count(0.25)
    rng = np.random.default_rng(7)
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    t0 = time.time()
    tiles = H.hctt_encode(w, k)
    del w
    log(f"encoded 8192x8192 in {time.time() - t0:.1f}s ({tiles.size} tile bytes)")
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    dt = torch.from_numpy(tiles).cuda()
    out = torch.empty(rows * cols, dtype=torch.bfloat16, device="cuda")
    launches = 10

    def step():
        for _ in range(launches):
            ctx.hctt_decode(dt, tiles.size, rows, cols, k, out, dtype=H.BF16, stream=sp)

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    check = None
    if O is not None:
        sub = 512
        rc, ref = O.hctt_decode_tensor(tiles[:(sub // 64) * (cols // 64) * H.hctt_tile_bytes(k)],
                                       sub, cols, k)
        got = out.view(rows, cols)[:sub].float().cpu().numpy()
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        check = float(np.abs(got - ref).max() / rms)
        log(f"spot check rows 0..{sub}: max|bf16 - oracle f32| = {check:.2e} x RMS")
    warm(step, args)
    T = Timed(torch, stream)
    e = T.start()
    for _ in range(args.steps):
        step()
    T.stop(e)
    torch.cuda.synchronize()
    ms_step = T.mean_s() * 1e3 / args.steps
    per = ms_step / 1e3 / launches
    out_b = rows * cols * 2
    flop = 256.0 * rows * cols
    cpu = None
    if not args.no_cpu and O is not None:
        sub = 1024
        part = tiles[:(sub // 64) * (cols // 64) * H.hctt_tile_bytes(k)]
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_budget:
            O.hctt_decode_tensor(part, sub, cols, k, nthreads=cpu_threads())
            reps += 1
        secs = time.perf_counter() - t0
        cpu = {"value": round(reps * sub * cols * 2 / secs / 1e9, 3), "unit": "GB/s",
               "cores": cpu_threads(), "kind": "port",
               "sample": f"{reps} decodes of rows 0..{sub} (2048 tiles: dequant + scatter + f32 "
                         f"Makhoul IDCT), bf16-equivalent output bytes, {cpu_threads()} threads, "
                         f"{secs:.1f} s"}
    return line("idct-8192", out_b / per / 1e9, ms_step, args, "f16-split-mfma/f32",
                "synthetic (8192x8192 N(0,0.02), seed 7)",
                {"rows": rows, "cols": cols, "rho": 0.25, "k": k, "tile_bytes": int(tiles.size),
                 "out_dtype": "bf16", "launches_per_step": launches},
                roofline("idct-8192", "hctt_decode_kernel<bf16>", tiles.size + out_b, per,
                         {"algorithmic_tflops": round(flop / per / 1e12, 1),
                          "issued_mfma": "v_mfma_f32_32x32x16_f16, 3 split passes, even/odd "
                                         "halves: 48 per tile"}),
                cpu, {"spot_check_max_err_over_rms": check})


def wl_hct3(args, torch, H, O):
    """Whole-tensor HCT3 spectral decode (GpuDecompressor::decompress_to_gpu)
    of one n x n (default 4096) N(0, 0.02) tensor encoded with the turbo defaults
    (retention 0.20, 4 fragments, essential ratio 0.20,
    crates/haagenti/src/pipeline/turbo.rs:88-96), the container resident in
    HBM, bf16 output."""
    import struct
    n = args.hct3_size
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    w = torch.randn(n, n, device="cuda", generator=g) * 0.02
    c = torch.empty_like(w)
    t0 = time.time()
    ctx.dct_2d(w, n, n, c, stream=sp)
    torch.cuda.synchronize()
    frags = H.CompressiveSpectralEncoder(4, 0.20).with_essential_ratio(0.20).encode_2d_from_dct(
        c.cpu().numpy(), n, n)
    del w, c
    # one container fragment: fragment 0's bitmap and every retained value
    f0 = frags[0][1]
    keep = struct.unpack_from("<I", f0, 12)[0]
    bm = n * n // 8
    payload = struct.pack("<I", keep) + f0[24:24 + bm] + f0[24 + bm:] + b"".join(d[8:] for _, d in frags[1:])
    data = struct.pack("<H", 1) + struct.pack("<HHQI", 0, 0, H.xxh3_64(payload), len(payload)) + payload
    log(f"encoded {n}x{n} in {time.time() - t0:.1f}s: {keep} coefficients, container {len(data) / 1e6:.1f} MB")
    d_data = torch.from_numpy(np.frombuffer(data, np.uint8).copy()).cuda()
    out = torch.empty(n * n, dtype=torch.bfloat16, device="cuda")
    dec = H.GpuDecompressor(ctx)

    def step():
        dec.decompress_device(data, d_data, [n, n], out, dtype=H.BF16, stream=sp)

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    check, cpu = None, None
    if O is not None:
        t0 = time.perf_counter()
        rc, ref = O.hct3_decode(data, [n, n])
        secs = time.perf_counter() - t0
        reps = 1
        assert rc == 0
        got = out.float().cpu().numpy()
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        check = float(np.abs(got - ref).max() / rms)
        log(f"full tensor: max|bf16 - oracle f32| = {check:.2e} x RMS")
        if not args.no_cpu:
            # more whole decodes until the budget is spent
            while secs < args.cpu_budget:
                t1 = time.perf_counter()
                O.hct3_decode(data, [n, n])
                secs += time.perf_counter() - t1
                reps += 1
            cpu = {"value": round(reps * n * n * 2 / secs / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                   "sample": f"{reps} full {n}x{n} decode(s) by the oracle (container scatter + the reference's "
                             f"FFT-based idct_2d in f32), bf16-equivalent output bytes, 1 thread, {secs:.1f} s"}
    warm(step, args)
    T = Timed(torch, stream)
    e = T.start()
    for _ in range(args.steps):
        step()
    T.stop(e)
    torch.cuda.synchronize()
    ms_step = T.mean_s() * 1e3 / args.steps
    per = ms_step / 1e3
    if args.dct_route != "dense":
        # the FFT route (the default at this size): bound by HBM; algorithmic
        # bytes = the container read once + the bf16 output written once
        alg = len(data) + n * n * 2
        achieved = alg / per / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(achieved / 8000.0, 4), "traffic": traffic_for(f"hct3-{n}-fft"),
                "kernel": ("dct_fft_rows_kernel x2 (Makhoul rows over an f32 Stockham FFT in LDS; the first "
                           "builds its rows from the fragments in LDS) + transpose_kernel x2 (the second "
                           "converting to bf16) + bitmap packing, row counts and their scan"),
                "avg_launch_us": round(per * 1e6, 1), "algorithmic_bytes_per_launch": alg,
                # the first row pass's f32 write, the first transpose and the second row pass (read +
                # write each), the last transpose's f32 read and bf16 write
                "f32_matrix_passes_bytes": 4 * n * n * 6 + 2 * n * n}
        dt = "f32-fft"
    else:
        flop = 4.0 * n ** 3          # the two dense n x n x n products of the transform
        achieved = flop / per / 1e12
        peak = 2500.0
        roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": traffic_for(f"hct3-{n}"),
                "kernel": ("dct_gemm_kernel x2 (hand-written split-f16 MFMA on the even / odd split of the "
                           "cosine bases: half-depth products, 2 + 3 passes, f32 accumulation; + butterfly, "
                           "bitmap scatter and the amax / scale passes)"),
                "avg_launch_us": round(per * 1e6, 1), "algorithmic_flop_per_launch": flop,
                "mfma_type": "f16", "mfma_flop_per_launch": 5 * n ** 3}
        dt = "f16-split-mfma/f32"
    return line(f"hct3-{n}", n * n * 2 / per / 1e9, ms_step, args, dt,
                f"synthetic ({n}x{n} N(0,0.02), torch seed 17, turbo defaults)",
                {"rows": n, "cols": n, "retention": 0.20, "coefficients": int(keep),
                 "container_bytes": len(data), "out_dtype": "bf16", "dct_route": args.dct_route}, roof, cpu,
                {"spot_check_max_err_over_rms": check})


def write_layer_files(H, L, shapes, d):
    """The layer's tensors as HCT v2 files (one per tensor, its LZ4 blocks
    with their XXH3 in the index: HctWriterV2), in d.  Returns, per file,
    (path, offset of its first block in the layer blob, payload bytes)."""
    out = []
    for T, (name, rows, cols) in zip(L["tensors"], shapes):
        sel = np.flatnonzero((L["out_off"] >= T["soff"]) & (L["out_off"] < T["soff"] + T["tlen"]))
        w = H.HctWriterV2(2, [rows, cols], int(L["out_cap"][sel[0]]))      # dtype 2 = BF16
        for j in sel:
            a = int(L["in_off"][j])
            w.add_block(L["blob"][a:a + int(L["in_len"][j])].tobytes(), int(L["out_cap"][j]))
        path = os.path.join(d, f"{name}.hct")
        with open(path, "wb") as f:
            f.write(w.finish())
        first = int(L["in_off"][sel[0]])
        out.append((path, first, int(L["in_off"][sel[-1]]) + int(L["in_len"][sel[-1]]) - first))
    return out


def wl_stream(args, torch, H, O):
    """Config 5 through the product pipeline (hh_pipeline_*: pinned staging,
    copy stream + compute stream ordered by events, double-buffered output
    slot), one seeded 70B layer encoding streamed --stream-layers times."""
    import haagenti_amd.pipeline as P
    rng = np.random.default_rng(70)
    rhos = rng.uniform(0.10, 0.50, len(L70B))
    ks = [H.hctt_retain_count(float(r)) for r in rhos]
    n_elem = sum(r * c for _, r, c in L70B)
    out_layer = n_elem * 2
    t0 = time.time()
    L = encode_layer(H, L70B, ks, 70, args.lz4_block)
    log(f"encoded one 70B layer in {time.time() - t0:.1f}s: {L['blob'].size / 1e6:.1f} MB "
        f"compressed, {L['scratch_bytes'] / 1e6:.1f} MB tile bytes; k = {ks}")
    ctx = new_ctx(H, args)
    nin = int(L["blob"].size)
    nb = int(L["in_off"].size)
    cfg = P.default_config()
    cfg.num_staging_buffers = 2
    cfg.max_blocks = nb
    cfg.staging_buffer_size = nin + 24 * nb + 256
    cfg.tile_scratch_size = L["scratch_bytes"]
    pool = P.MemoryPool(ctx, 2 * cfg.staging_buffer_size + cfg.tile_scratch_size + (16 << 20))
    pipe = P.DecompressionPipeline(ctx, pool, cfg)
    # compressed layer in pinned host memory (copied to the device from there)
    host = P.PinnedBuffer(nin)
    host.copy_from_host(L["blob"])
    files, maps, rpool = None, [], None
    if args.from_file:
        # the layer as HCT v2 files, memory-mapped; each layer's payloads are
        # read by host threads straight into the pipeline's next staging
        # buffer while the previous layers copy and decode
        import concurrent.futures as cf
        import mmap
        import tempfile
        d = tempfile.mkdtemp(prefix="hct70b_", dir=os.environ.get("TMPDIR", "/tmp"))
        files = write_layer_files(H, L, L70B, d)
        for path, first, nbytes in files:
            f = open(path, "rb")
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            r = H.HctReaderV2(mm[:])                  # header checksum, block index
            r.validate_checksums()
            start = r.data_offset()
            assert mm[start:start + nbytes] == L["blob"][first:first + nbytes].tobytes()
            maps.append((f, mm, start, first, nbytes))
        rpool = cf.ThreadPoolExecutor(max_workers=8)
        log(f"wrote {len(files)} HCT v2 files ({sum(x[2] for x in files) / 1e6:.1f} MB of blocks) to {d}")

    def read_layer(dst):
        jobs = []
        for _, mm, start, first, nbytes in maps:
            step = 8 << 20
            for o in range(0, nbytes, step):
                n = min(step, nbytes - o)
                jobs.append(rpool.submit(np.copyto, dst[first + o:first + o + n],
                                         np.frombuffer(mm, np.uint8, n, start + o)))
        for j in jobs:
            j.result()

    slot = [[torch.empty(r * c, dtype=torch.bfloat16, device="cuda") for _, r, c in L70B] for _ in range(2)]
    tabs = (L["in_off"], L["in_len"], L["out_off"], L["out_cap"])
    read_s = [0.0]

    def run(nlayers, timed):
        tickets = []
        for l in range(nlayers):
            src = host.as_slice()
            if args.from_file:
                r0 = time.perf_counter()
                st = pipe.next_staging()
                read_layer(st)
                read_s[0] += time.perf_counter() - r0 if timed else 0.0
                src = st[:nin]
            desc = [(t["tlen"], t["rows"], t["cols"], t["k"], slot[l % 2][i]) for i, t in enumerate(L["tensors"])]
            tickets.append(pipe.submit(src, *tabs, tensors=desc, dtype=H.BF16))
        return tickets

    tk = run(2, False)                        # correctness pass (checked below)
    for t in tk:
        pipe.wait(t)                          # raises on any failed block
    check = None
    if O is not None:
        T0 = L["tensors"][1]                  # k (1024 x 8192), first rows
        sub = 256
        tb = H.hctt_tile_bytes(T0["k"])
        comp, kinds, _ = O.lz4_decompress_batch(L["blob"], L["in_off"], L["in_len"], L["out_off"], L["out_cap"],
                                                L["scratch_bytes"], nthreads=cpu_threads())
        rc, ref = O.hctt_decode_tensor(comp[T0["soff"]:T0["soff"] + (sub // 64) * (T0["cols"] // 64) * tb], sub,
                                       T0["cols"], T0["k"])
        got = slot[1][1].view(T0["rows"], T0["cols"])[:sub].float().cpu().numpy()
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        check = float(np.abs(got - ref).max() / rms)
        assert (kinds == 0).all()
        del comp
        log(f"spot check layer 1 / k rows 0..{sub}: max|bf16 - oracle f32| = {check:.2e} x RMS")
    for _ in range(max(1, args.warmup // 10)):
        for t in run(2, False):
            pipe.wait(t)
    pipe.finish()
    pipe.reset_stats()
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    tk = run(args.stream_layers, True)
    times = [pipe.times(t) for t in tk]
    pipe.finish()
    wall = time.perf_counter() - w0
    st = pipe.stats()
    e2e_ms = times[-1].decode_end_ms - times[0].h2d_start_ms
    dec_s = st.decompress_time_ns / st.units / 1e9
    h2d_s = st.transfer_time_ns / st.units / 1e9
    value = out_layer / dec_s / 1e9
    e2e = out_layer * args.stream_layers / (e2e_ms / 1e3) / 1e9
    h2d_gbs = nin / h2d_s / 1e9
    # copy of layer l + 1 under the decode of layer l, from the event times
    hidden = [max(0.0, min(times[l + 1].h2d_end_ms, times[l].decode_end_ms) -
                  max(times[l + 1].h2d_start_ms, times[l].decode_start_ms)) /
              (times[l].decode_end_ms - times[l].decode_start_ms) for l in range(len(times) - 1)]
    overlap = float(np.mean(hidden))
    file_info = None
    if args.from_file:
        file_info = {"files": len(files), "host_read_gbs": round(nin * args.stream_layers / read_s[0] / 1e9, 2),
                     "source": "HCT v2 files (mmap, page cache) -> pinned staging (in place) -> H2D"}
        log(f"from files: host reads {file_info['host_read_gbs']} GB/s")
        for f, mm, *_ in maps:
            mm.close()
            f.close()
        rpool.shutdown()
        import shutil
        shutil.rmtree(os.path.dirname(files[0][0]), ignore_errors=True)
    log(f"per layer: decode {dec_s * 1e3:.2f} ms ({value:.0f} GB/s out), H2D {h2d_s * 1e3:.2f} ms "
        f"({h2d_gbs:.1f} GB/s), end to end {e2e_ms / args.stream_layers:.2f} ms/layer "
        f"({e2e:.0f} GB/s out); decode hidden under the next copy: {overlap:.3f}; wall {wall:.2f}s")
    cpu = None
    if not args.no_cpu and O is not None:
        reps, secs, ne = cpu_layer_decode(O, L, args.cpu_budget, tensor_subset=[1, 2])
        cpu = {"value": round(reps * ne * 2 / secs / 1e9, 3), "unit": "GB/s", "cores": cpu_threads(),
               "kind": "port",
               "sample": f"{reps} x LZ4 of the whole 70B layer + tile decode of its k and v tensors "
                         f"({ne} elements), {cpu_threads()} threads, {secs:.1f} s"}
    # the route's launches (as hh_pipeline_submit plans them: every block of
    # this encoding holds whole tiles) and its algorithmic bytes: compressed
    # in, bf16 out, and the tile bytes of the two-launch tensors written and
    # read back through the scratch
    fused_ks = {"auto": {t["k"] for t in L["tensors"] if t["k"] >= 1024}, "two-launch": set(),
                "fused": {t["k"] for t in L["tensors"]}}[args.pipeline_route]
    two_launch_tile_bytes = sum(t["tlen"] for t in L["tensors"] if t["k"] not in fused_ks)
    rest_ks = [t["k"] for t in L["tensors"] if t["k"] not in fused_ks]
    lz4_name = LZ4_KERNEL_NAMES[("seq" if min(rest_ks) < 1024 else "ring4") if args.lz4_decoder == "auto"
                                else args.lz4_decoder].split("<")[0] if rest_ks else None
    stream_kernels = " + ".join((["hctt_lz4_fused_kernel<bf16>"] if fused_ks else []) +
                                ([lz4_name, "hctt_decode_kernel<bf16>"] if rest_ks else []))
    res = line("llama70b-stream", value, e2e_ms / args.stream_layers, args,
               "f16-split-mfma/f32",
               "synthetic (one seeded 70B layer encoding streamed %d times)" % args.stream_layers,
               {"layers": args.stream_layers, "elements_per_layer": n_elem,
                "rho": [round(float(r), 4) for r in rhos], "k": ks,
                "compressed_bytes_per_layer": nin, "out_dtype": "bf16",
                "source": file_info["source"] if file_info else "pinned host memory (hh_pinned_alloc)",
                "value_is": "decode-only (events around the unit's decode launches on the pipeline's compute stream)",
                "runtime": "hh_pipeline_* (copy stream + compute stream, 2 staging slots)"},
               roofline("llama70b-stream", stream_kernels, nin + out_layer + 2 * two_launch_tile_bytes, dec_s,
                        {"fused_tensors": [t["name"] for t in L["tensors"] if t["k"] in fused_ks]}),
               cpu,
               {"end_to_end_gbs": round(e2e, 2), "h2d_gbs": round(h2d_gbs, 2),
                "decode_ms_per_layer": round(dec_s * 1e3, 3),
                "h2d_ms_per_layer": round(h2d_s * 1e3, 3),
                "overlap_fraction": round(overlap, 3), "from_file": file_info,
                "spot_check_max_err_over_rms": check})
    pipe.close()
    pool.close()
    host.close()
    return res


def wl_copy(args, torch, H, O):
    """1 GiB streaming copy with the library's hand-written copy kernel
    (hh_hbm_copy), the runtime's copy timed beside it."""
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    launches = 10

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        T = Timed(torch, stream)
        e = T.start()
        for _ in range(args.steps * launches):
            fn()
        T.stop(e)
        torch.cuda.synchronize()
        return T.mean_s() / (args.steps * launches)

    per = timed(lambda: ctx.hbm_copy(b, a, n, stream=sp))
    ok = bool(torch.equal(a, b))
    per_rt = timed(lambda: b.copy_(a))
    log(f"hand-written copy {2 * n / per / 1e9:.0f} GB/s in+out (bytes equal: {ok}); "
        f"runtime copy {2 * n / per_rt / 1e9:.0f} GB/s")
    return line("hbm-copy", 2 * n / per / 1e9, per * 1e3 * launches, args, "u8",
                "synthetic (1 GiB device buffer)",
                {"bytes_read": n, "bytes_written": n, "runtime_copy_gbs": round(2 * n / per_rt / 1e9, 1)},
                roofline("hbm-copy", "hh_hbm_copy (hand-written streaming copy, calibration)", 2 * n, per), None)


def wl_xxh3(args, torch, H, O):
    nb = 4096
    srcs, pick, blob, in_off, in_len = config2_blocks(H)
    ctx = new_ctx(H, args)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    d_in = torch.from_numpy(blob.copy()).cuda()
    d_off, d_len = devtab(torch, in_off), devtab(torch, in_len)
    d_out = torch.zeros(nb, dtype=torch.int64, device="cuda")
    launches = 10

    def step():
        for _ in range(launches):
            ctx.xxh3_64_batch(d_in, d_in.numel(), d_off, d_len, nb, d_out, stream=sp)

    step()                                   # correctness pass (checked below)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy().view(np.uint64)
    exact = all(int(got[j]) == H.xxh3_64(blob[in_off[j]:in_off[j] + in_len[j]].tobytes())
                for j in range(0, nb, 97))
    log(f"spot check of every 97th block vs the host XXH3: {exact}")
    warm(step, args)
    T = Timed(torch, stream)
    e = T.start()
    for _ in range(args.steps):
        step()
    T.stop(e)
    torch.cuda.synchronize()
    ms_step = T.mean_s() * 1e3 / args.steps
    per = ms_step / 1e3 / launches
    in_b = int(blob.size)
    cpu = None
    if not args.no_cpu and O is not None:
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_budget:
            O.xxh3_64_batch(blob, in_off, in_len, cpu_threads())
            reps += 1
        secs = time.perf_counter() - t0
        cpu = {"value": round(reps * in_b / secs / 1e9, 3), "unit": "GB/s", "cores": cpu_threads(),
               "kind": "port",
               "sample": f"{reps} x all {nb} blocks ({in_b} bytes), {cpu_threads()} threads, {secs:.1f} s"}
    return line("xxh3-256mib", in_b / per / 1e9, ms_step, args, "u64",
                "synthetic (the lz4-256mib compressed blocks)",
                {"blocks": nb, "in_bytes": in_b, "launches_per_step": launches},
                roofline("xxh3-256mib", "xxh3_batch_kernel", in_b, per), cpu,
                {"spot_check_exact": exact})


WORKLOADS = {"llama3-8b-layer": wl_llama3_8b_layer, "xxh3-256mib": wl_xxh3, "int4-4096": wl_int4, "lz4-256mib": wl_lz4,
             "idct-8192": wl_idct, "llama70b-stream": wl_stream, "hbm-copy": wl_copy, "hct3-4096": wl_hct3}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=20,
                    help="untimed steps first (the clocks settle within ~50 ms of load)")
    ap.add_argument("--workload", default="llama3-8b-layer", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=32, help="llama3-8b-layer: layers per step")
    ap.add_argument("--layers-per-launch", type=int, default=4,
                    help="llama3-8b-layer, fused path: consecutive layers decoded by one hh_hctt_decode_lz4_fused "
                         "call (their 7 tensors each; one launch for up to 32 tensors)")
    ap.add_argument("--stream-layers", type=int, default=80, help="llama70b-stream: layers")
    ap.add_argument("--distinct", type=int, default=2, help="distinct encoded layers")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--from-file", action="store_true",
                    help="llama70b-stream: read each layer from HCT v2 files (mmap) into pinned staging")
    ap.add_argument("--kernel-sample", type=int, default=8,
                    help="llama3-8b-layer: per-kernel events on every n-th layer of the timed steps")
    ap.add_argument("--path", choices=["fused", "two-launch"], default="fused",
                    help="llama3-8b-layer: fused LZ4 + tile launches (hh_hctt_decode_lz4_fused) "
                         "or the LZ4 and tile launches through a scratch buffer (hh_hctt_decode_lz4_batch)")
    ap.add_argument("--hct3-size", type=int, default=4096, help="hct3-4096: side of the square tensor")
    ap.add_argument("--dct-route", default="auto", choices=["auto", "dense", "fft"],
                    help="whole-matrix transform route of hct3-4096 (the context's HH_OPT_DCT_ROUTE)")
    ap.add_argument("--lz4-decoder", default="auto", choices=sorted(LZ4_KERNEL_NAMES),
                    help="LZ4 block decoder of the batched LZ4 launches (the context's HH_OPT_LZ4_DECODER)")
    ap.add_argument("--pipeline-route", default="auto", choices=["auto", "two-launch", "fused"],
                    help="llama70b-stream: how the pipeline decodes a layer's tensors (the context's "
                         "HH_OPT_PIPELINE_ROUTE): dense tensors in the fused launch (auto), two launches "
                         "for every tensor, or the fused launch for every tensor")
    ap.add_argument("--lz4-block", type=int, default=16384,
                    help="LZ4 block size in bytes before rounding down to whole tiles "
                         "(the reference HctWriter default is 16 KiB)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the decode runs on "
              "a single MI355X; across GPUs each would decode its own tensors or 64-aligned slabs, "
              "with nothing exchanged).", file=sys.stderr)
        sys.exit(2)
    if args.layers_per_launch not in (1, 2, 4) or args.layers % args.layers_per_launch:
        print("--layers-per-launch is 1, 2 or 4 (a launch takes up to 32 tensors, 7 per layer) and divides "
              "--layers", file=sys.stderr)
        sys.exit(2)
    import torch
    import haagenti_amd as H
    torch.cuda.set_device(0)
    O = oracle()
    res = WORKLOADS[args.workload](args, torch, H, O)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
