"""hh_hctt_decode_lz4_fused: LZ4 blocks of whole tiles and their tiles in one
launch, the tile bytes kept in LDS (HctReader::decompress_all,
crates/haagenti-hct/src/tensor.rs:417-515, with the per-tile decode of
GpuDecompressor::decompress_batch_to_gpu, crates/haagenti-cuda/src/
decompress.rs:282-293, fused).

The tile arithmetic is the same code as the two-launch path
(hh_hctt_decode_lz4_batch), so every output is compared bit for bit with
that path (itself checked against the oracle at 1e-3 x RMS in
test_gpu_llama_layers.py), and one tensor per layer against the oracle
directly.  A block that fails or decodes short gets the batched LZ4 kernel's
status record, and its tiles report HH_ERR_CORRUPTED_DATA with zero output
while every other tile is unaffected."""
import numpy as np
import pytest

import gpu_util as G
import layer_util as LU
import oracle_lib as O
from test_gpu_llama_layers import check_against_oracle, decode

pytestmark = pytest.mark.gpu


# Every test runs with each block decoder the fused kernel can use (the
# context's HH_OPT_LZ4_DECODER): the one-sequence ring decoder (the fused
# entry's default) and the sequence-batched decoder.
@pytest.fixture(autouse=True, params=["ring4", "seq"])
def lz4_decoder(request):
    G.ctx().set_lz4_decoder(request.param)
    yield request.param
    G.ctx().set_lz4_decoder("auto")


def H():
    import haagenti_amd as h
    return h


def encode_fixed(Hm, shapes, ks, seed, tpb):
    """A layer whose every tensor is cut into blocks of tpb whole tiles (the
    last block of a tensor the rest), in the layout encode_layer returns."""
    rng = np.random.default_rng(seed)
    comp = Hm.Lz4Compressor()
    parts, in_off, in_len, out_off, out_cap, tensors = [], [], [], [], [], []
    pos = spos = 0
    for (name, rows, cols), k in zip(shapes, ks):
        w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        tiles = Hm.hctt_encode(w, k)
        tb = Hm.hctt_tile_bytes(k)
        for s in range(0, tiles.size, tpb * tb):
            chunk = tiles[s:s + tpb * tb]
            c = comp.compress(chunk.tobytes())
            parts.append(c)
            in_off.append(pos)
            in_len.append(len(c))
            out_off.append(spos + s)
            out_cap.append(chunk.size)
            pos += len(c)
        tensors.append(dict(name=name, rows=rows, cols=cols, k=k, soff=spos, tiles=tiles))
        spos += tiles.size
    return dict(blob=np.frombuffer(b"".join(parts), np.uint8), in_off=np.array(in_off, np.uint64),
                in_len=np.array(in_len, np.uint32), out_off=np.array(out_off, np.uint64),
                out_cap=np.array(out_cap, np.uint32), tensors=tensors, scratch_bytes=spos)


def fused(L, dtype, tpb, blob=None, expect_rc=0):
    Hm = H()
    T = G.torch()
    d_in = G.dev(L["blob"] if blob is None else blob)
    in_off, in_len = G.dev(L["in_off"]), G.dev(L["in_len"])
    n = L["in_off"].size
    status = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    tdt = {Hm.F32: T.float32, Hm.BF16: T.bfloat16, Hm.F16: T.float16}[dtype]
    outs, tst, desc = [], [], []
    for t in L["tensors"]:
        o = T.full((t["rows"] * t["cols"],), 7.0, dtype=tdt, device="cuda")
        s = T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda")
        outs.append(o)
        tst.append(s)
        desc.append((t["rows"], t["cols"], t["k"], o, s))
    print(f"[fused] {len(desc)} tensors, {n} blocks of {tpb} tiles, dtype {dtype}", flush=True)
    rc = G.ctx().hctt_decode_lz4_fused(d_in, d_in.numel(), in_off, in_len, n, status, desc, tpb, dtype,
                                       stream=G.stream())
    assert rc == expect_rc
    G.sync()
    st = np.frombuffer(status.cpu().numpy().tobytes(), dtype=np.dtype(
        [("code", "<i4"), ("detail", "<i4"), ("position", "<u8"), ("required", "<u8"), ("written", "<u8")]))
    return outs, st, tst


def test_llama3_8b_layer_fused_equals_two_launch_path():
    Hm = H()
    T = G.torch()
    k = Hm.hctt_retain_count(0.3)
    L = LU.encode_layer(Hm, LU.L8B, [k] * 7, seed=8)
    tpb = 16384 // Hm.hctt_tile_bytes(k)
    assert tpb == 13
    for dtype in (Hm.F32, Hm.BF16):
        fo, st, fs = fused(L, dtype, tpb)
        assert (st["code"] == 0).all() and (st["written"] == L["out_cap"]).all()
        assert all((s.cpu().numpy() == 0).all() for s in fs)
        bo, codes, scratch, _ = decode(L, dtype)
        del scratch
        assert (codes == 0).all()
        for t, a, b in zip(L["tensors"], fo, bo):
            assert T.equal(a.view(T.int32 if dtype == Hm.F32 else T.int16),
                           b.view(T.int32 if dtype == Hm.F32 else T.int16)), (t["name"], dtype)
        if dtype == Hm.F32:
            check_against_oracle(dict(tensors=L["tensors"][1:2]), fo[1:2])
        del fo, bo


_LAYERS = {}


def test_four_llama3_8b_layers_in_one_launch():
    # the bench's default step: four layers' 28 tensors in one fused launch
    # (their blocks in one buffer, each later layer's offsets shifted), bit
    # for bit the same outputs, tile statuses and block records as one
    # launch per layer
    Hm = H()
    T = G.torch()
    k = Hm.hctt_retain_count(0.3)
    tpb = 16384 // Hm.hctt_tile_bytes(k)
    if not _LAYERS:
        _LAYERS["L"] = [LU.encode_layer(Hm, LU.L8B, [k] * 7, seed=s) for s in (21, 22, 23, 24)]
    Ls = _LAYERS["L"]
    base = np.cumsum([0] + [L["blob"].size for L in Ls[:-1]]).astype(np.uint64)
    allL = dict(blob=np.concatenate([L["blob"] for L in Ls]),
                in_off=np.concatenate([L["in_off"] + b for L, b in zip(Ls, base)]),
                in_len=np.concatenate([L["in_len"] for L in Ls]),
                tensors=[t for L in Ls for t in L["tensors"]])
    assert len(allL["tensors"]) == 28
    fo, st, fs = fused(allL, Hm.BF16, tpb)
    assert (st["code"] == 0).all()
    b0 = 0
    for i, L in enumerate(Ls):
        lo, lst, ls = fused(L, Hm.BF16, tpb)
        nb = L["in_off"].size
        assert np.array_equal(lst, st[b0:b0 + nb])
        b0 += nb
        for j in range(7):
            assert T.equal(lo[j].view(T.int16), fo[7 * i + j].view(T.int16)), (i, j)
            assert T.equal(ls[j], fs[7 * i + j]), (i, j)
        del lo, ls
    del fo, fs


def test_mixed_retention_fixed_blocks_vs_oracle():
    Hm = H()
    rng = np.random.default_rng(41)
    shapes = [("a", 512, 1024), ("b", 1024, 512), ("c", 256, 2048), ("d", 640, 384)]
    ks = [Hm.hctt_retain_count(float(r)) for r in rng.uniform(0.10, 0.50, len(shapes))]
    tpb = min(Hm.FUSED_BLOCK_BYTES // Hm.hctt_tile_bytes(k) for k in ks)
    L = encode_fixed(Hm, shapes, ks, seed=42, tpb=tpb)
    fo, st, fs = fused(L, Hm.F32, tpb)
    assert (st["code"] == 0).all()
    assert all((s.cpu().numpy() == 0).all() for s in fs)
    check_against_oracle(L, fo)
    # the same tiles through the two-launch path: bit-identical
    bo, codes, scratch, _ = decode(L, Hm.F32)
    assert (codes == 0).all()
    T = G.torch()
    for a, b in zip(fo, bo):
        assert T.equal(a.view(T.int32), b.view(T.int32))


def test_failed_and_short_blocks_poison_only_their_tiles():
    Hm = H()
    T = G.torch()
    shapes = [("a", 256, 512), ("b", 512, 256)]
    ks = [Hm.hctt_retain_count(0.3), Hm.hctt_retain_count(0.2)]
    tpb = 5
    L = encode_fixed(Hm, shapes, ks, seed=43, tpb=tpb)
    n = L["in_off"].size
    blob = L["blob"].copy()
    # block 2: a corrupted offset field is far past the output (CORRUPTED);
    # block n - 3: the stream ends early (decodes short or fails)
    bad = [2, n - 3]
    lens = L["in_len"].copy()
    o2 = int(L["in_off"][2])
    blob[o2 + 1:o2 + int(lens[2])] ^= 0x5A
    lens[n - 3] = max(1, lens[n - 3] // 3)
    L2 = dict(L, in_len=lens)
    fo, st, fs = fused(L2, Hm.F32, tpb, blob=blob)
    # the records are the batched LZ4 kernel's for the same blocks and sizes
    d_in = G.dev(blob)
    ref_st = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    scratch = T.zeros(L["scratch_bytes"], dtype=T.uint8, device="cuda")
    G.ctx().lz4_decompress_batch(d_in, d_in.numel(), G.dev(L["in_off"]), G.dev(lens), scratch,
                                 G.dev(L["out_off"]), G.dev(L["out_cap"]), n, ref_st, stream=G.stream())
    G.sync()
    ref = np.frombuffer(ref_st.cpu().numpy().tobytes(), dtype=st.dtype)
    for f in ("code", "detail", "position", "required"):
        assert np.array_equal(st[f], ref[f]), f
    short = [b for b in bad if ref["code"][b] != 0 or ref["written"][b] < L["out_cap"][b]]
    assert len(short) == 2
    # map blocks to tiles and check the poisoning
    bo, codes, sc, _ = decode(L, Hm.F32)
    blk = 0
    for t, a, b, s in zip(L["tensors"], fo, bo, fs):
        nt = (t["rows"] // 64) * (t["cols"] // 64)
        stt = s.cpu().numpy()
        a_np = a.cpu().numpy().reshape(t["rows"] // 64, 64, t["cols"] // 64, 64)
        b_np = b.cpu().numpy().reshape(t["rows"] // 64, 64, t["cols"] // 64, 64)
        tpr = t["cols"] // 64
        for j in range((nt + tpb - 1) // tpb):
            g = blk + j
            good = int(st["written"][g]) if st["code"][g] == 0 else 0
            tb = Hm.hctt_tile_bytes(t["k"])
            for tt in range(j * tpb, min(nt, (j + 1) * tpb)):
                r, c = divmod(tt, tpr)
                lo, hi = (tt - j * tpb) * tb, (tt - j * tpb + 1) * tb
                if hi <= good:      # every byte of the tile produced
                    assert stt[tt] == 0
                    assert np.array_equal(a_np[r, :, c, :].view(np.int32), b_np[r, :, c, :].view(np.int32))
                elif lo >= good:    # none: all zero bytes
                    assert g in bad
                    assert stt[tt] == Hm.CORRUPTED_DATA, (t["name"], g, tt)
                    assert (a_np[r, :, c, :] == 0).all()
        blk += (nt + tpb - 1) // tpb


def test_argument_errors():
    Hm = H()
    k = Hm.hctt_retain_count(0.3)
    L = encode_fixed(Hm, [("a", 128, 128)], [k], seed=44, tpb=2)
    assert L["in_off"].size == 2
    T = G.torch()
    d_in = G.dev(L["blob"])
    st = T.zeros(64, dtype=T.uint8, device="cuda")
    o = T.empty(128 * 128, dtype=T.float32, device="cuda")
    args = (d_in, d_in.numel(), G.dev(L["in_off"]), G.dev(L["in_len"]))
    assert G.ctx().hctt_decode_lz4_fused(*args, 3, st, [(128, 128, k, o)], 2) == Hm.INVALID_ARGUMENT
    assert G.ctx().hctt_decode_lz4_fused(*args, 1, st, [(128, 128, k, o)], 14) == Hm.UNSUPPORTED
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(100, 128, k, o)], 2) == Hm.INVALID_ARGUMENT
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(64, (1 << 24) + 64, k, o)], 2) == Hm.INVALID_ARGUMENT
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(128, 128, k, o)], 2) == Hm.OK
    # the per-tensor entry (hh_hctt_decode_lz4_fused_tpb): a zero count, a
    # block over HH_FUSED_BLOCK_BYTES, a block total that does not match
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(128, 128, k, o)], [0]) == Hm.INVALID_ARGUMENT
    assert G.ctx().hctt_decode_lz4_fused(*args, 1, st, [(128, 128, k, o)], [14]) == Hm.UNSUPPORTED
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(128, 128, k, o), (64, 64, k, o)], [2, 1]) == \
        Hm.INVALID_ARGUMENT
    assert G.ctx().hctt_decode_lz4_fused(*args, 2, st, [(128, 128, k, o)], [2]) == Hm.OK


def both_paths(L, dtype, tpb, blob=None, lens=None):
    """The same blocks through the fused call and the two-launch call:
    outputs, tile statuses and block records (the two-launch path's LZ4
    records are hh_lz4_decompress_batch's)."""
    L2 = dict(L)
    if blob is not None:
        L2["blob"] = blob
    if lens is not None:
        L2["in_len"] = lens
    fo, st, fs = fused(L2, dtype, tpb)
    bo, codes, scratch, bs = decode(L2, dtype)
    del scratch
    return fo, st, fs, bo, codes, bs


def assert_same(T, dtype, fo, fs, bo, bs):
    Hm = H()
    view = T.int32 if dtype == Hm.F32 else T.int16
    for i, (a, b, sa, sb) in enumerate(zip(fo, bo, fs, bs)):
        assert T.equal(a.view(view), b.view(view)), i
        assert T.equal(sa, sb), i


@pytest.mark.parametrize("ntensors", [32, 33, 40])
def test_many_tensors_small_blocks_f16(ntensors):
    # up to 32 tensors in one launch, more in launches of at most 32; blocks
    # of one and of three tiles, f16 output
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(51)
    base = [(64, 64), (128, 64), (64, 192), (192, 128), (64, 64), (256, 64), (128, 128), (64, 320), (320, 64),
            (128, 192), (64, 128), (192, 64), (64, 64), (128, 256), (64, 448), (256, 128), (64, 64), (192, 192),
            (128, 64), (64, 256)]
    shapes = [("t%d" % i, r, c) for i, (r, c) in enumerate((base + base[::-1])[:ntensors])]
    ks = [Hm.hctt_retain_count(float(r)) for r in rng.uniform(0.10, 0.50, len(shapes))]
    for tpb in (1, 3):
        L = encode_fixed(Hm, shapes, ks, seed=52 + tpb, tpb=tpb)
        fo, st, fs, bo, codes, bs = both_paths(L, Hm.F16, tpb)
        assert (st["code"] == 0).all() and (codes == 0).all()
        assert all((s.cpu().numpy() == 0).all() for s in fs)
        assert_same(T, Hm.F16, fo, fs, bo, bs)


def test_large_retention_tiles():
    # k = 4096 (2,816-byte tiles, 5 per block) and k = 3000 (7 per block):
    # fewer waves fit the LDS next to the block buffers (a wave's area holds
    # a table of k entries)
    Hm = H()
    T = G.torch()
    for k, shape in ((4096, ("a", 320, 256)), (3000, ("b", 256, 448))):
        tpb = Hm.FUSED_BLOCK_BYTES // Hm.hctt_tile_bytes(k)
        L = encode_fixed(Hm, [shape], [k], seed=k, tpb=tpb)
        fo, st, fs, bo, codes, bs = both_paths(L, Hm.F32, tpb)
        assert (st["code"] == 0).all() and (codes == 0).all()
        assert_same(T, Hm.F32, fo, fs, bo, bs)
        check_against_oracle(L, fo)


def test_failed_blocks_one_per_workgroup():
    # 188 blocks of two tiles over up to 256 workgroups: one block per
    # workgroup, whose waves then mostly wait on that block's decoder; ten
    # corrupted blocks poison all of their tiles, exactly as the two-launch
    # path does
    Hm = H()
    T = G.torch()
    shapes = [("a", 1024, 512), ("b", 512, 1024), ("c", 768, 640)]
    ks = [Hm.hctt_retain_count(0.3), Hm.hctt_retain_count(0.2), Hm.hctt_retain_count(0.4)]
    tpb = 2
    L = encode_fixed(Hm, shapes, ks, seed=61, tpb=tpb)
    n = L["in_off"].size
    assert n == 188
    rng = np.random.default_rng(62)
    bad = sorted(rng.choice(n, 10, replace=False).tolist())
    blob = L["blob"].copy()
    for b in bad:
        o = int(L["in_off"][b])
        blob[o + 1:o + int(L["in_len"][b])] ^= 0x5A
    fo, st, fs, bo, codes, bs = both_paths(L, Hm.F32, tpb, blob=blob)
    assert (st["code"][bad] != 0).all() and (np.delete(st["code"], bad) == 0).all()
    assert np.array_equal(st["code"], codes)
    assert_same(T, Hm.F32, fo, fs, bo, bs)
    # and the corrupted tiles are zeros
    corrupted = sum(int((s.cpu().numpy() == Hm.CORRUPTED_DATA).sum()) for s in fs)
    assert corrupted == tpb * len(bad)  # every tensor's tile count is even: full blocks
    for t, a, s in zip(L["tensors"], fo, fs):
        a = a.cpu().numpy().reshape(t["rows"] // 64, 64, t["cols"] // 64, 64)
        for tt in np.nonzero(s.cpu().numpy() == Hm.CORRUPTED_DATA)[0]:
            r, c = divmod(int(tt), t["cols"] // 64)
            assert (a[r, :, c, :] == 0).all()


def test_fewer_tiles_than_workgroups():
    # two tiles in all: two workgroups, one tile each, sharing the one block
    Hm = H()
    T = G.torch()
    k = Hm.hctt_retain_count(0.25)
    L = encode_fixed(Hm, [("a", 64, 128)], [k], seed=71, tpb=2)
    assert L["in_off"].size == 1
    fo, st, fs, bo, codes, bs = both_paths(L, Hm.BF16, 2)
    assert (st["code"] == 0).all()
    assert_same(T, Hm.BF16, fo, fs, bo, bs)


def test_per_tensor_tiles_per_block():
    # every tensor cut into blocks of floor(16352 / its tile bytes) whole
    # tiles (one writer per tensor with a whole-tile block size), retention
    # 0.18-0.42: the sparse tensor's blocks are a few hundred short LZ4
    # sequences each (4-byte matches thousands of bytes back); then the same
    # layer with a truncated block of the sparse tensor
    Hm = H()
    T = G.torch()
    shapes = [("a", 512, 1024), ("b", 256, 1536), ("c", 1024, 512), ("d", 384, 640)]
    ks = [Hm.hctt_retain_count(r) for r in (0.18, 0.42, 0.25, 0.33)]
    tpb = [Hm.FUSED_BLOCK_BYTES // Hm.hctt_tile_bytes(k) for k in ks]
    assert len(set(tpb)) == 4
    L = LU.encode_layer(Hm, shapes, ks, seed=71, block_bytes=Hm.FUSED_BLOCK_BYTES)
    fo, st, fs, bo, codes, bs = both_paths(L, Hm.F32, tpb)
    assert (st["code"] == 0).all() and (codes == 0).all()
    assert all((s.cpu().numpy() == 0).all() for s in fs)
    assert_same(T, Hm.F32, fo, fs, bo, bs)
    check_against_oracle(L, fo)
    bad = 3
    lens = L["in_len"].copy()
    lens[bad] //= 2
    fo, st, fs, bo, codes, bs = both_paths(L, Hm.BF16, tpb, lens=lens)
    assert st["code"][bad] != 0 and codes[bad] == st["code"][bad]
    assert (np.delete(st["code"], bad) == 0).all()
    assert_same(T, Hm.BF16, fo, fs, bo, bs)
    assert (fs[0].cpu().numpy()[bad * tpb[0]:(bad + 1) * tpb[0]] == Hm.CORRUPTED_DATA).all()


def test_bounded_waits_give_up_cleanly():
    # every wait of the fused kernel gives up after the context's poll limit
    # (normally 2^24; here 1, so the waits at the start of a workgroup's run,
    # before its first block's bytes are decoded, run out): the waves leave
    # through the workgroup's abort word, and every block record and tile
    # status of a workgroup that gave up reports HH_ERR_DEVICE (workgroup g
    # of G holds blocks g, g + G, ...; a workgroup that never waited long
    # enough decodes as usual); the kernel ends, and the next call decodes
    # normally
    Hm = H()
    k = Hm.hctt_retain_count(0.3)
    tpb = 13
    L = encode_fixed(Hm, [("a", 1024, 1024), ("b", 512, 2048)], [k, k], seed=81, tpb=tpb)
    G.ctx().set_option(Hm.OPT_FUSED_POLL_LIMIT, 1)
    try:
        _, st, fs = fused(L, Hm.F32, tpb)
    finally:
        G.ctx().set_option(Hm.OPT_FUSED_POLL_LIMIT, 0)
    codes = st["code"]
    print(f"[fused] spin limit 1: {int((codes == Hm.DEVICE).sum())} of {codes.size} block records HH_ERR_DEVICE",
          flush=True)
    assert set(np.unique(codes).tolist()) <= {Hm.OK, Hm.DEVICE}
    assert (codes == Hm.DEVICE).any()
    nb = codes.size
    grid = min(G.torch().cuda.get_device_properties(0).multi_processor_count, nb)
    for g in range(grid):
        assert len(set(codes[g::grid].tolist())) == 1   # a workgroup's blocks all alike
    # each block's tiles report what its record reports
    blk = 0
    for t, s in zip(L["tensors"], fs):
        s = s.cpu().numpy()
        ntiles = (t["rows"] // 64) * (t["cols"] // 64)
        for j in range(0, ntiles, tpb):
            want = Hm.DEVICE if codes[blk] == Hm.DEVICE else 0
            assert (s[j:j + tpb] == want).all()
            blk += 1
    assert blk == nb
    fo, st, fs = fused(L, Hm.F32, tpb)
    assert (st["code"] == 0).all()
    assert all((s.cpu().numpy() == 0).all() for s in fs)
    check_against_oracle(L, fo)
