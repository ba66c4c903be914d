"""One decoder layer's LZ4-compressed HCT-T tensors in one call
(hh_hctt_decode_lz4_batch: HctReader::decompress_all then
GpuDecompressor::decompress_batch_to_gpu, crates/haagenti-hct/src/
tensor.rs:417-515 and crates/haagenti-cuda/src/decompress.rs:282-293):
bit-identical to the two batched calls it queues, within 1e-3 x RMS of the
oracle's decode of the same tiles, LZ4 status records equal to the
oracle's, and a corrupt block reported without disturbing the other
tensors."""
import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O

pytestmark = pytest.mark.gpu
TOL = 1e-3


def H():
    import haagenti_amd as h
    return h


def layer(seed=4):
    """Three tensors with their own k, LZ4 blocks of 3 whole tiles."""
    Hm = H()
    rng = np.random.default_rng(seed)
    blocks, tensors, spos = [], [], 0
    for rows, cols, k in [(128, 192, 1228), (64, 256, 410), (192, 64, 2048)]:
        w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        tiles = Hm.hctt_encode(w, k)
        tb = Hm.hctt_tile_bytes(k)
        for s in range(0, tiles.size, 3 * tb):
            chunk = tiles[s:s + 3 * tb].tobytes()
            blocks.append((O.lz4_compress_block(chunk)[0], spos + s, len(chunk)))
        tensors.append(dict(rows=rows, cols=cols, k=k, soff=spos, tiles=tiles))
        spos += tiles.size
    return blocks, tensors, spos


def match_offset_positions(c):
    """Byte positions of every match offset in a raw LZ4 block (the block
    format of crates/haagenti-lz4/src/block.rs:261-366)."""
    i, out = 0, []
    while i < len(c):
        t = c[i]
        i += 1
        ll = t >> 4
        if ll == 15:
            while True:
                x = c[i]
                i += 1
                ll += x
                if x != 255:
                    break
        i += ll
        if i >= len(c):
            break
        out.append(i)
        i += 2
        if t & 15 == 15:
            while c[i] == 255:
                i += 1
            i += 1
    return out


def device_tables(blocks):
    T = G.torch()
    comp = b"".join(c for c, _, _ in blocks)
    in_off = np.cumsum([0] + [len(c) for c, _, _ in blocks[:-1]]).astype(np.int64)
    tabs = [G.dev(np.frombuffer(comp, np.uint8)), len(comp), T.from_numpy(in_off).cuda(),
            T.from_numpy(np.array([len(c) for c, _, _ in blocks], np.int32)).cuda(),
            T.from_numpy(np.array([o for _, o, _ in blocks], np.int64)).cuda(),
            T.from_numpy(np.array([n for _, _, n in blocks], np.int32)).cuda()]
    return comp, tabs


def run(blocks, tensors, scratch_len, fused, dtype, stale=None, tile_status=False):
    """stale: bytes the scratch holds before the call (an earlier layer's
    tiles); tile_status: also return every tensor's per-tile status."""
    Hm = H()
    T = G.torch()
    comp, (d_in, in_total, d_off, d_len, d_oo, d_oc) = device_tables(blocks)
    if stale is None:
        scratch = T.zeros(scratch_len, dtype=T.uint8, device="cuda")
    else:
        scratch = G.dev(np.ascontiguousarray(stale[:scratch_len]))
    status = T.zeros(len(blocks) * 32, dtype=T.uint8, device="cuda")
    tdt = T.float32 if dtype == Hm.F32 else T.bfloat16
    outs = [T.empty(t["rows"] * t["cols"], dtype=tdt, device="cuda") for t in tensors]
    tst = [T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda") for t in tensors]
    desc = [(scratch.data_ptr() + t["soff"], t["tiles"].size, t["rows"], t["cols"], t["k"], o, s)
            for t, o, s in zip(tensors, outs, tst)]
    ctx = G.ctx()
    if fused:
        ctx.hctt_decode_lz4_batch(d_in, in_total, d_off, d_len, scratch, d_oo, d_oc, len(blocks), status, desc,
                                  dtype=dtype, stream=G.stream())
    else:
        assert ctx.lz4_decompress_batch(d_in, in_total, d_off, d_len, scratch, d_oo, d_oc, len(blocks), status,
                                        stream=G.stream()) == Hm.OK
        ctx.hctt_decode_batch(desc, dtype=dtype, stream=G.stream())
    G.sync()
    codes = status.cpu().numpy().view(np.int32).reshape(-1, 8)
    if tile_status:
        return [o.cpu() for o in outs], codes, scratch.cpu().numpy(), [s.cpu().numpy() for s in tst]
    return [o.cpu() for o in outs], codes, scratch.cpu().numpy()


@pytest.mark.parametrize("dtype_name", ["F32", "BF16"])
def test_fused_layer_call_equals_two_calls_and_oracle(dtype_name):
    Hm = H()
    dtype = getattr(Hm, dtype_name)
    blocks, tensors, slen = layer()
    a, ca, sa = run(blocks, tensors, slen, True, dtype)
    b, cb, sb = run(blocks, tensors, slen, False, dtype)
    assert (ca[:, 0] == 0).all() and np.array_equal(ca, cb)
    for t in tensors:
        assert np.array_equal(sa[t["soff"]:t["soff"] + t["tiles"].size], t["tiles"])   # LZ4 bit-exact
    for t, x, y in zip(tensors, a, b):
        assert np.array_equal(x.view(G.torch().int16).numpy() if dtype == Hm.BF16 else x.numpy(),
                              y.view(G.torch().int16).numpy() if dtype == Hm.BF16 else y.numpy())
        rc, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        assert rc == O.OK
        got = x.float().numpy().reshape(t["rows"], t["cols"])
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        tol = TOL if dtype == Hm.F32 else 2 ** -7     # bf16: RNE of the f32 result
        assert np.abs(got - ref).max() <= tol * (rms if dtype == Hm.F32 else np.abs(ref).max())


@pytest.mark.parametrize("cut", ["truncated", "zero_offset"])
def test_fused_layer_call_reports_a_corrupt_block(cut):
    # The scratch still holds an earlier layer's valid tiles (the same layer
    # here, so every stale bitmap has the right popcount).  The reference
    # returns Err and no output for the layer (tensor.rs:506-515); here the
    # failed block's output range is zeroed, so every tile it covers reports
    # CORRUPTED and decodes to zeros instead of to the stale bytes.
    Hm = H()
    blocks, tensors, slen = layer(seed=9)
    stale = np.concatenate([t["tiles"] for t in tensors])
    bad = 2                                   # the first block of the second tensor
    c, o, n = blocks[bad]
    if cut == "truncated":
        blocks[bad] = (c[:len(c) // 2], o, n)     # the reference reports UnexpectedEof
    else:
        # the last match's offset set to zero: the reference reports
        # "invalid zero offset" after most of the block has been written
        offs = match_offset_positions(c)
        assert offs
        b = bytearray(c)
        b[offs[-1]] = b[offs[-1] + 1] = 0
        blocks[bad] = (bytes(b), o, n)
    outs, codes, scratch, tst = run(blocks, tensors, slen, True, Hm.F32, stale=stale, tile_status=True)
    for j, (cb, _, nb) in enumerate(blocks):
        _, e = O.lz4_decompress_block(cb, nb)
        assert codes[j, 0] == e.kind
    assert codes[bad, 0] != Hm.OK and (np.delete(codes[:, 0], bad) == 0).all()
    # the failed block's range of the scratch reads as zeros
    assert (scratch[o:o + n] == 0).all()
    t = tensors[1]
    tb = Hm.hctt_tile_bytes(t["k"])
    first, last = (o - t["soff"]) // tb, (o + n - 1 - t["soff"]) // tb
    assert (tst[1][first:last + 1] == Hm.CORRUPTED_DATA).all()
    assert (np.delete(tst[1], np.arange(first, last + 1)) == Hm.OK).all()
    assert (tst[0] == Hm.OK).all() and (tst[2] == Hm.OK).all()
    x = outs[1].numpy().reshape(t["rows"], t["cols"])
    tpr = t["cols"] // 64
    for tt in range(first, last + 1):
        r, cc = divmod(tt, tpr)
        assert (x[64 * r:64 * r + 64, 64 * cc:64 * cc + 64] == 0).all()
    for t, x in zip([tensors[0], tensors[2]], [outs[0], outs[2]]):
        _, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(x.numpy().reshape(t["rows"], t["cols"]) - ref).max() <= TOL * rms


def test_batch_of_more_than_thirty_two_tensors_with_empty_ones():
    # more tensors than one launch takes (32), empty ones among them: every
    # tensor decoded once, each against the oracle, tile statuses all OK
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(12)
    half = [(64, 128), (0, 64), (128, 64), (64, 64), (0, 0), (64, 192), (128, 128), (64, 64),
            (192, 64), (64, 0), (64, 256), (128, 192), (64, 64), (128, 64), (64, 320), (192, 128),
            (0, 128), (64, 64), (256, 64), (64, 128), (128, 128), (64, 192)]
    shapes = half + half[::-1]
    descs, refs, outs, tsts = [], [], [], []
    keep = []
    for i, (rows, cols) in enumerate(shapes):
        k = int(rng.integers(1, 4097))
        if rows and cols:
            w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
            tiles = Hm.hctt_encode(w, k)
            _, ref = O.hctt_decode_tensor(tiles, rows, cols, k)
        else:
            tiles, ref = np.zeros(1, np.uint8), None
        d = G.dev(tiles)
        out = T.full((max(rows * cols, 1),), float("nan"), dtype=T.float32, device="cuda")
        st = T.full((max((rows // 64) * (cols // 64), 1),), -1, dtype=T.int32, device="cuda")
        keep.append(d)
        descs.append((d, tiles.size, rows, cols, k, out, st))
        refs.append(ref)
        outs.append(out)
        tsts.append(st)
    G.ctx().hctt_decode_batch(descs, dtype=Hm.F32, stream=G.stream())
    G.sync()
    for (rows, cols), ref, out, st in zip(shapes, refs, outs, tsts):
        if ref is None:
            assert out.isnan().all() and (st.cpu().numpy() == -1).all()     # untouched
            continue
        assert (st.cpu().numpy() == Hm.OK).all()
        got = out.cpu().numpy().reshape(rows, cols)
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        assert np.abs(got - ref).max() <= TOL * rms
