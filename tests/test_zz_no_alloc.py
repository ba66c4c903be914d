"""hh_hctt_decode_lz4_batch_noalloc (the layer decode with the library's own
tile-byte array, for callers that cannot allocate) against
hh_hctt_decode_lz4_batch with a caller scratch: identical outputs, LZ4
status records and tile statuses, over two calls in a row (a full
Llama-3-8B layer, then a smaller layer), and the size / argument errors."""
import numpy as np
import pytest

import gpu_util as G
import layer_util as LU

pytestmark = pytest.mark.gpu


def H():
    import haagenti_amd as h
    return h


def small_layer(Hm, seed):
    shapes = [("a", 128, 192), ("b", 64, 256), ("c", 192, 64), ("d", 64, 64)]
    ks = [1228, 410, 2048, 77]
    return LU.encode_layer(Hm, shapes, ks, seed=seed, block_bytes=4096)


def tables(L):
    return [G.dev(L["blob"])] + [G.dev(L[x]) for x in ("in_off", "in_len", "out_off", "out_cap")]


def decode_both(L, dtype):
    """The layer through both entry points; returns their (outputs, block
    status bytes, tile statuses)."""
    Hm = H()
    T = G.torch()
    d_in, d_off, d_len, d_oo, d_oc = tables(L)
    n = L["in_off"].size
    tdt = {Hm.F32: T.float32, Hm.BF16: T.bfloat16, Hm.F16: T.float16}[dtype]
    res = []
    for noalloc in (False, True):
        outs = [T.full((t["rows"] * t["cols"],), 7.0, dtype=tdt, device="cuda") for t in L["tensors"]]
        tst = [T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda")
               for t in L["tensors"]]
        status = T.full((n * 32,), 0x5A, dtype=T.uint8, device="cuda")
        print(f"[noalloc] {'noalloc' if noalloc else 'scratch'} call: {len(outs)} tensors, {n} blocks, "
              f"{L['scratch_bytes']} tile bytes", flush=True)
        if noalloc:
            desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o, s)
                    for t, o, s in zip(L["tensors"], outs, tst)]
            rc = G.ctx().hctt_decode_lz4_batch_noalloc(d_in, d_in.numel(), d_off, d_len, d_oo, d_oc, n, status,
                                                       desc, dtype=dtype, stream=G.stream())
            assert rc == Hm.OK
        else:
            scratch = T.empty(L["scratch_bytes"], dtype=T.uint8, device="cuda")
            desc = [(scratch.data_ptr() + t["soff"], t["tiles"].size, t["rows"], t["cols"], t["k"], o, s)
                    for t, o, s in zip(L["tensors"], outs, tst)]
            G.ctx().hctt_decode_lz4_batch(d_in, d_in.numel(), d_off, d_len, scratch, d_oo, d_oc, n, status, desc,
                                          dtype=dtype, stream=G.stream())
        G.sync()
        res.append(([o.view(T.int16 if dtype != Hm.F32 else T.int32).cpu().numpy() for o in outs],
                    status.cpu().numpy(), [s.cpu().numpy() for s in tst]))
    return res


def assert_same(a, b):
    (oa, sa, ta), (ob, sb, tb) = a, b
    assert np.array_equal(sa, sb)
    assert (sa.view(np.int32)[0::8] == 0).all()
    for x, y in zip(oa, ob):
        assert np.array_equal(x, y)
    for x, y in zip(ta, tb):
        assert np.array_equal(x, y) and (x == 0).all()


def test_noalloc_layer_decode_equals_scratch_decode_twice():
    Hm = H()
    k = Hm.hctt_retain_count(0.3)
    big = LU.encode_layer(Hm, LU.L8B, [k] * 7, seed=31)
    assert big["scratch_bytes"] <= Hm.NOALLOC_SCRATCH_BYTES
    a, b = decode_both(big, Hm.BF16)
    assert_same(a, b)
    del big
    small = small_layer(Hm, seed=32)              # the second call is smaller
    a, b = decode_both(small, Hm.F32)
    assert_same(a, b)


def test_noalloc_rejects_oversized_and_misplaced_inputs():
    Hm = H()
    T = G.torch()
    L = small_layer(Hm, seed=33)
    d_in, d_off, d_len, d_oo, d_oc = tables(L)
    n = L["in_off"].size
    status = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    out = T.empty(128 * 192, dtype=T.float32, device="cuda")
    ctx = G.ctx()
    # more tile bytes than the array holds: nothing is launched
    rc = ctx.hctt_decode_lz4_batch_noalloc(d_in, d_in.numel(), d_off, d_len, d_oo, d_oc, n, status,
                                           [(Hm.NOALLOC_SCRATCH_BYTES + 1, 128, 192, 1228, out)], dtype=Hm.F32,
                                           stream=G.stream())
    assert rc == Hm.BUFFER_TOO_SMALL
    # blocks whose output lies past the packed tiles of the tensors given
    # (only the first tensor here) are reported and write nothing
    t0 = L["tensors"][0]
    rc = ctx.hctt_decode_lz4_batch_noalloc(d_in, d_in.numel(), d_off, d_len, d_oo, d_oc, n, status,
                                           [(t0["tiles"].size, t0["rows"], t0["cols"], t0["k"], out)],
                                           dtype=Hm.F32, stream=G.stream())
    assert rc == Hm.OK
    G.sync()
    codes = status.cpu().numpy().view(np.int32)[0::8]
    inside = (L["out_off"] + L["out_cap"]) <= t0["tiles"].size
    assert inside.any() and (~inside).any()
    assert (codes[inside] == Hm.OK).all() and (codes[~inside] == Hm.INVALID_ARGUMENT).all()


def test_noalloc_call_allocates_no_device_memory():
    # The entry point's defining property: a call, even the first on a
    # fresh context, leaves the device's free memory unchanged (kernels are
    # loaded first through the shared context; loading code objects is the
    # runtime's, once per process).
    Hm = H()
    T = G.torch()
    L = small_layer(Hm, seed=34)
    d_in, d_off, d_len, d_oo, d_oc = tables(L)
    n = L["in_off"].size
    outs = [T.empty(t["rows"] * t["cols"], dtype=T.float32, device="cuda") for t in L["tensors"]]
    desc = [(t["tiles"].size, t["rows"], t["cols"], t["k"], o) for t, o in zip(L["tensors"], outs)]
    status = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    assert G.ctx().hctt_decode_lz4_batch_noalloc(d_in, d_in.numel(), d_off, d_len, d_oo, d_oc, n, status, desc,
                                                 dtype=Hm.F32, stream=G.stream()) == Hm.OK
    G.sync()
    ctx = Hm.HipContext(0)
    try:
        G.sync()
        free0 = T.cuda.mem_get_info()[0]
        rc = ctx.hctt_decode_lz4_batch_noalloc(d_in, d_in.numel(), d_off, d_len, d_oo, d_oc, n, status, desc,
                                               dtype=Hm.F32, stream=G.stream())
        G.sync()
        free1 = T.cuda.mem_get_info()[0]
        print(f"[noalloc] free device memory before {free0} after {free1}", flush=True)
        assert rc == Hm.OK
        assert free1 == free0
        assert (status.cpu().numpy().view(np.int32)[0::8] == 0).all()
    finally:
        ctx.close()
