"""Streaming decode runtime on the GPU: MemoryPool and PinnedBuffer
(crates/haagenti-cuda/src/memory.rs:156-340) and DecompressionPipeline
(crates/haagenti-cuda/src/pipeline.rs:87-320) streaming Llama-70B-shaped
layers from pinned host memory into a double-buffered output slot, each
layer checked against the oracle, the copy of layer l + 1 observed under
the decode of layer l."""
import numpy as np
import pytest

import gpu_util as G
import layer_util as LU
import oracle_lib as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


def H():
    import haagenti_amd as h
    return h


def P():
    import haagenti_amd.pipeline as p
    return p


def test_memory_pool_first_fit_and_coalescing():
    Hm, Pm = H(), P()
    pool = Pm.MemoryPool(G.ctx(), 1 << 20)
    assert pool.total_size() == 1 << 20 and pool.allocated() == 0
    a = pool.allocate(1000)                      # 256-byte pieces
    b = pool.allocate(4096)
    c = pool.allocate(300)
    assert (b.ptr - a.ptr, c.ptr - b.ptr) == (1024, 4096)
    assert pool.allocated() == 1024 + 4096 + 512
    pool.recycle(b)
    s = pool.stats()
    assert s.free_buffers == 2 and s.largest_free == (1 << 20) - 1024 - 4096 - 512
    assert s.available == (1 << 20) - 1024 - 512
    d = pool.allocate(2048)                      # first fit: b's hole
    assert d.ptr == b.ptr
    pool.recycle(a)
    pool.recycle(d)
    pool.recycle(c)                              # everything coalesces back
    s = pool.stats()
    assert s.allocated == 0 and s.free_buffers == 1 and s.free_buffer_bytes == 1 << 20
    big = pool.allocate(1 << 20)
    with pytest.raises(Hm.HaagentiError) as ei:
        pool.allocate(1)                         # OutOfMemory
    assert ei.value.code == Hm.OUT_OF_MEMORY
    with pytest.raises(Hm.HaagentiError):
        pool.recycle(Pm.GpuBuffer(big.ptr + 256, 1, pool))   # not a piece start
    pool.recycle(big)
    pool.close()


def test_pool_pieces_are_zeroed_on_request():
    Pm = P()
    pool = Pm.MemoryPool(G.ctx(), 1 << 16)
    a = pool.allocate(5000, zero=False)
    G.h2d(a.ptr, np.full(5000, 0xAB, np.uint8))
    assert (G.d2h(a.ptr, 5000) == 0xAB).all()
    pool.recycle(a)
    b = pool.allocate(5000, zero=True)           # the same piece, cleared
    assert b.ptr == a.ptr and (G.d2h(b.ptr, 5000) == 0).all()
    pool.recycle(b)
    pool.close()


def test_pinned_buffer():
    Hm, Pm = H(), P()
    b = Pm.PinnedBuffer(1024)
    b.copy_from_host(bytes([1, 2, 3, 4]))
    assert b.size() == 4 and bytes(b.as_slice()) == bytes([1, 2, 3, 4])
    with pytest.raises(Hm.HaagentiError):
        b.copy_from_host(bytes(2048))            # SizeMismatch
    b.close()


def _layer_tables(L):
    return L["in_off"], L["in_len"], L["out_off"], L["out_cap"]


def test_pipeline_streams_70b_layers_with_overlap():
    Hm, Pm = H(), P()
    T = G.torch()
    rng = np.random.default_rng(75)
    ks_a = [Hm.hctt_retain_count(float(r)) for r in rng.uniform(0.10, 0.50, 7)]
    ks_b = [Hm.hctt_retain_count(float(r)) for r in rng.uniform(0.10, 0.50, 7)]
    LA = LU.encode_layer(Hm, LU.L70B, ks_a, seed=76)
    LB = LU.encode_layer(Hm, LU.L70B, ks_b, seed=77)
    layers = [LA, LB, LA]
    # compressed layers in pinned host memory
    pins = []
    for L in (LA, LB):
        pb = Pm.PinnedBuffer(L["blob"].size)
        pb.copy_from_host(L["blob"])
        pins.append(pb)
    cfg = Pm.default_config()
    cfg.num_staging_buffers = 2
    cfg.max_blocks = max(L["in_off"].size for L in (LA, LB))
    cfg.staging_buffer_size = max(L["blob"].size for L in (LA, LB)) + 24 * cfg.max_blocks + 256
    cfg.tile_scratch_size = max(L["scratch_bytes"] for L in (LA, LB))
    pool = Pm.MemoryPool(G.ctx(), 2 * cfg.staging_buffer_size + cfg.tile_scratch_size + (16 << 20))
    pipe = Pm.DecompressionPipeline(G.ctx(), pool, cfg)
    # the double-buffered output slot: two sets of the layer's tensors (f32)
    slots = [[T.empty(r * c, dtype=T.float32, device="cuda") for _, r, c in LU.L70B] for _ in range(2)]
    tst = [[T.full(((r // 64) * (c // 64),), -1, dtype=T.int32, device="cuda") for _, r, c in LU.L70B]
           for _ in range(2)]

    def submit(i):
        L = layers[i]
        src = pins[0 if L is LA else 1].as_slice()
        desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o, s)
                for t, o, s in zip(L["tensors"], slots[i % 2], tst[i % 2])]
        print(f"[pipeline] submit layer {i}: {src.size} bytes, {L['in_off'].size} blocks", flush=True)
        return pipe.submit(src, *_layer_tables(L), tensors=desc, dtype=Hm.F32)

    def check(i):
        L = layers[i]
        for t, o, s in zip(L["tensors"], slots[i % 2], tst[i % 2]):
            assert (s.cpu().numpy() == 0).all()
            rc, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
            assert rc == O.OK
            got = o.cpu().numpy().reshape(t["rows"], t["cols"])
            rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
            err = float(np.abs(got - ref).max())
            print(f"[pipeline] layer {i} {t['name']}: {err / rms:.2e} x RMS", flush=True)
            assert err <= TOL * rms

    # hold the copy stream (a bounded clock spin, ~20 ms) so that both units
    # are enqueued before the first copy starts: the overlap below then does
    # not depend on how fast this host returns from submit
    copy_s, _ = pipe.streams
    with T.cuda.stream(T.cuda.ExternalStream(copy_s)):
        T.cuda._sleep(50_000_000)
    t0 = submit(0)
    t1 = submit(1)                                # copy of layer 1 under the decode of layer 0
    pipe.wait(t0)
    check(0)
    t2 = submit(2)                                # back into slot 0, after layer 0 was read
    pipe.wait(t1)
    check(1)
    pipe.wait(t2)
    check(2)
    tm = [pipe.times(t) for t in (t0, t1, t2)]
    for i, t in enumerate(tm):
        print(f"[pipeline] layer {i}: h2d {t.h2d_start_ms:.3f}-{t.h2d_end_ms:.3f} ms, "
              f"decode {t.decode_start_ms:.3f}-{t.decode_end_ms:.3f} ms", flush=True)
        assert t.h2d_start_ms <= t.h2d_end_ms <= t.decode_start_ms <= t.decode_end_ms
    # overlap: layer 1's copy runs while layer 0 decodes
    assert tm[1].h2d_start_ms < tm[0].decode_end_ms and tm[1].h2d_end_ms > tm[0].decode_start_ms
    st = pipe.stats()
    assert st.units == 3 and st.blocks_processed == sum(L["in_off"].size for L in layers)
    assert st.bytes_read == sum(L["blob"].size for L in layers)
    assert st.bytes_output == 3 * 4 * sum(r * c for _, r, c in LU.L70B)
    pipe.finish()
    pipe.close()
    pool.close()


def test_pipeline_pageable_and_in_place_staging_and_errors():
    # a small layer through both host paths (pageable source copied into
    # staging; data written straight into next_staging()), a corrupt block
    # reported by wait() with its index, and finish() after that
    Hm, Pm = H(), P()
    T = G.torch()
    shapes = [("a", 128, 192), ("b", 64, 256), ("c", 192, 64)]
    L = LU.encode_layer(Hm, shapes, [1228, 410, 2048], seed=78, block_bytes=4096)
    cfg = Pm.default_config()
    cfg.staging_buffer_size = 1 << 20
    cfg.tile_scratch_size = 1 << 20
    cfg.max_blocks = 64
    pipe = Pm.DecompressionPipeline(G.ctx(), None, cfg)
    refs = []
    for t in L["tensors"]:
        _, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        refs.append(ref)

    def run(src, blob_tables=None):
        outs = [T.empty(r * c, dtype=T.float32, device="cuda") for _, r, c in shapes]
        desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o) for t, o in zip(L["tensors"], outs)]
        tk = pipe.submit(src, *(blob_tables or _layer_tables(L)), tensors=desc, dtype=Hm.F32)
        return tk, outs

    tk, outs = run(L["blob"].copy())                         # pageable
    pipe.wait(tk)
    st = pipe.next_staging()                                 # in place
    st[:L["blob"].size] = L["blob"]
    tk2, outs2 = run(st[:L["blob"].size])
    pipe.wait(tk2)
    for o, o2, t, ref in zip(outs, outs2, L["tensors"], refs):
        a = o.cpu().numpy().reshape(t["rows"], t["cols"])
        assert np.array_equal(a, o2.cpu().numpy().reshape(t["rows"], t["cols"]))
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(a - ref).max() <= TOL * rms
    # a truncated block: wait() names it
    bad = 3
    il = L["in_len"].copy()
    il[bad] //= 2
    tk3, _ = run(L["blob"].copy(), (L["in_off"], il, L["out_off"], L["out_cap"]))
    with pytest.raises(Hm.HaagentiError) as ei:
        pipe.wait(tk3)
    a = int(L["in_off"][bad])
    _, e = O.lz4_decompress_block(L["blob"][a:a + int(il[bad])].tobytes(), int(L["out_cap"][bad]))
    assert ei.value.code == e.kind and ei.value.block == bad
    # raw LZ4 into a caller buffer, no tensors, failure reported by finish()
    dst = T.zeros(L["scratch_bytes"], dtype=T.uint8, device="cuda")
    tk4 = pipe.submit(L["blob"].copy(), *_layer_tables(L), lz4_out=dst, lz4_out_cap=dst.numel())
    pipe.wait(tk4)
    assert np.array_equal(dst.cpu().numpy(), np.concatenate([t["tiles"] for t in L["tensors"]]))
    pipe.submit(L["blob"].copy(), L["in_off"], il, L["out_off"], L["out_cap"], lz4_out=dst,
                lz4_out_cap=dst.numel())
    with pytest.raises(Hm.HaagentiError) as ei:
        pipe.finish()
    assert ei.value.block == bad
    pipe.finish()                                            # nothing pending any more
    # an invalid tensor (rows not a multiple of 64) fails the submit before
    # anything is enqueued; the slot is reused by the next unit as if the
    # call had not happened
    outs = [T.full((r * c,), 3.0, dtype=T.float32, device="cuda") for _, r, c in shapes]
    desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o) for t, o in zip(L["tensors"], outs)]
    bad_desc = list(desc)
    bad_desc[1] = (L["tensors"][1]["tiles"].size, 65, 256, 410, outs[1])
    with pytest.raises(Hm.HaagentiError) as ei:
        pipe.submit(L["blob"].copy(), *_layer_tables(L), tensors=bad_desc, dtype=Hm.F32)
    assert ei.value.code == Hm.INVALID_ARGUMENT
    G.sync()
    assert all((o.cpu().numpy() == 3.0).all() for o in outs)   # nothing ran
    tk5 = pipe.submit(L["blob"].copy(), *_layer_tables(L), tensors=desc, dtype=Hm.F32)
    pipe.wait(tk5)
    for o, t, ref in zip(outs, L["tensors"], refs):
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(o.cpu().numpy().reshape(t["rows"], t["cols"]) - ref).max() <= TOL * rms
    pipe.close()


def test_pipeline_blocks_across_tile_boundaries():
    # each tensor written with HctWriter's default block size (16 KiB chunks
    # of its tile bytes, tiles cut between blocks: tensor.rs:556-561): the
    # LZ4 output lands in the scratch at block offsets inside tiles
    Hm, Pm = H(), P()
    T = G.torch()
    shapes = [("a", 256, 512), ("b", 512, 256)]
    ks = [Hm.hctt_retain_count(0.3), Hm.hctt_retain_count(0.22)]
    rng = np.random.default_rng(91)
    comp = Hm.Lz4Compressor()
    parts, in_off, in_len, out_off, out_cap, tens = [], [], [], [], [], []
    pos = spos = 0
    for (name, r, c), k in zip(shapes, ks):
        tiles = Hm.hctt_encode((rng.standard_normal((r, c), dtype=np.float32) * np.float32(0.02)), k)
        assert tiles.size % 16384 != 0 and 16384 % Hm.hctt_tile_bytes(k) != 0
        for s in range(0, tiles.size, 16384):
            chunk = tiles[s:s + 16384]
            cb = comp.compress(chunk.tobytes())
            parts.append(cb)
            in_off.append(pos)
            in_len.append(len(cb))
            out_off.append(spos + s)
            out_cap.append(chunk.size)
            pos += len(cb)
        tens.append(dict(name=name, rows=r, cols=c, k=k, tiles=tiles))
        spos += tiles.size
    blob = np.frombuffer(b"".join(parts), np.uint8)
    cfg = Pm.default_config()
    cfg.staging_buffer_size = 1 << 20
    cfg.tile_scratch_size = 1 << 20
    cfg.max_blocks = 64
    pipe = Pm.DecompressionPipeline(G.ctx(), None, cfg)
    outs = [T.empty(t["rows"] * t["cols"], dtype=T.float32, device="cuda") for t in tens]
    tst = [T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda") for t in tens]
    desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o, s) for t, o, s in zip(tens, outs, tst)]
    tk = pipe.submit(blob.copy(), np.array(in_off, np.uint64), np.array(in_len, np.uint32),
                     np.array(out_off, np.uint64), np.array(out_cap, np.uint32), tensors=desc, dtype=Hm.F32)
    pipe.wait(tk)
    for t, o, s in zip(tens, outs, tst):
        assert (s.cpu().numpy() == 0).all()
        rc, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        assert rc == O.OK
        got = o.cpu().numpy().reshape(t["rows"], t["cols"])
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(got - ref).max() <= TOL * rms
    pipe.close()


def test_pipeline_routes_agree_bit_for_bit():
    # one unit of mixed retention through the three routes of
    # hh_pipeline_submit (HH_OPT_PIPELINE_ROUTE): two launches for every
    # tensor; the fused launch for k >= 1024 (auto); the fused launch for
    # every tensor.  Outputs, tile statuses and block records agree bit for
    # bit, also with damaged blocks: tensor b's first block cut to one byte
    # (UnexpectedEof) and its second to half (a stream that ends cleanly
    # decodes short: the rest of its tile bytes read as zeros on every
    # route), and tensor c's first block cut by 7 bytes.  Under auto the
    # fused launch takes a and c, whose blocks come first in the staged
    # table; wait() still names the first failing block in the caller's
    # order.
    Hm, Pm = H(), P()
    T = G.torch()
    shapes = [("a", 128, 256), ("b", 192, 128), ("c", 64, 512), ("d", 128, 128)]
    ks = [1228, 410, 2048, 700]
    L = LU.encode_layer(Hm, shapes, ks, seed=93, block_bytes=4096)
    soff = np.cumsum([0] + [t["tiles"].size for t in L["tensors"]])
    tens = np.searchsorted(soff[1:], L["out_off"], side="right")
    b0, b1 = (int(x) for x in np.nonzero(tens == 1)[0][:2])   # tensor b (k = 410): its two blocks
    c0 = int(np.nonzero(tens == 2)[0][0])                       # tensor c (k = 2048), later in the table
    assert b0 < b1 < c0
    il = L["in_len"].copy()
    il[b0] = 1
    il[b1] //= 2
    il[c0] -= 7
    cfg = Pm.default_config()
    cfg.staging_buffer_size = 1 << 20
    cfg.tile_scratch_size = 1 << 20
    cfg.max_blocks = 64
    ctx = G.ctx()
    pipe = Pm.DecompressionPipeline(ctx, None, cfg)
    got = {}
    try:
        for route in ("two-launch", "auto", "fused"):
            ctx.set_pipeline_route(route)
            for dt, tdt in ((Hm.F32, T.float32), (Hm.BF16, T.bfloat16)):
                for tables in ((L["in_off"], L["in_len"], L["out_off"], L["out_cap"]),
                               (L["in_off"], il, L["out_off"], L["out_cap"])):
                    outs = [T.full((r * c,), 7, dtype=tdt, device="cuda") for _, r, c in shapes]
                    tst = [T.full(((r // 64) * (c // 64),), -1, dtype=T.int32, device="cuda") for _, r, c in shapes]
                    desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o, s)
                            for t, o, s in zip(L["tensors"], outs, tst)]
                    tk = pipe.submit(L["blob"].copy(), *tables, tensors=desc, dtype=dt)
                    failed = None
                    try:
                        pipe.wait(tk)
                    except Hm.HaagentiError as ex:
                        failed = (ex.code, ex.block, ex.status.detail, ex.status.position, ex.status.required)
                    key = (dt, tables[1] is il)
                    res = ([o.view(T.int16 if tdt == T.bfloat16 else T.int32).cpu().numpy() for o in outs],
                           [s.cpu().numpy() for s in tst], failed)
                    print(f"[routes] {route} dtype {dt} damaged {key[1]}: failed {failed}", flush=True)
                    if key not in got:
                        got[key] = res
                        continue
                    ref = got[key]
                    assert res[2] == ref[2]
                    for x, y in zip(res[0], ref[0]):
                        assert np.array_equal(x, y)
                    for x, y in zip(res[1], ref[1]):
                        assert np.array_equal(x, y)
    finally:
        ctx.set_pipeline_route("auto")
    # the clean unit decodes every tile, within the tolerance of the oracle
    assert got[(Hm.F32, False)][2] is None
    assert all((s == 0).all() for s in got[(Hm.F32, False)][1])
    for t, o in zip(L["tensors"], got[(Hm.F32, False)][0]):
        _, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(o.view(np.float32).reshape(t["rows"], t["cols"]) - ref).max() <= TOL * rms
    # the damaged unit: wait() names block b0 with the oracle's record
    code, block = got[(Hm.F32, True)][2][:2]
    assert block == b0
    a = int(L["in_off"][b0])
    _, e = O.lz4_decompress_block(L["blob"][a:a + int(il[b0])].tobytes(), int(L["out_cap"][b0]))
    assert code == e.kind
    # every tile of b (both its blocks damaged) and c's first two tiles
    # (its first block) report CORRUPTED_DATA with zero output; a and d decode
    st, out = got[(Hm.F32, True)][1], got[(Hm.F32, True)][0]
    assert (st[0] == 0).all() and (st[3] == 0).all()
    assert (st[1] == Hm.CORRUPTED_DATA).all() and (out[1] == 0).all()
    assert (st[2][:2] == Hm.CORRUPTED_DATA).all() and (st[2][2:] == 0).all()
    assert (out[2].reshape(64, 512)[:, :128] == 0).all()
    pipe.close()
