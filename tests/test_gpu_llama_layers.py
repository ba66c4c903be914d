"""Whole decoder layers at their real shapes through one
hh_hctt_decode_lz4_batch call (HctReader::decompress_all per tensor,
crates/haagenti-hct/src/tensor.rs:506-515, then per tile dequantize_int4,
crates/haagenti/src/testing/quantization.rs:82-131, the bitmap scatter and
idct_2d, crates/haagenti-core/src/dct.rs:311-337):

  * a Llama-3-8B layer (q,o 4096x4096; k,v 1024x4096; gate,up 14336x4096;
    down 4096x14336), 30 % retention (k = 1228), 13-tile 15,652-byte LZ4
    blocks: the LZ4 output bit-identical to the tile bytes, every tensor's
    f32 decode within 1e-3 x RMS of the oracle, and the bf16 decode equal to
    the round-to-nearest-even of the f32 decode for every tensor;
  * a Llama-70B layer (q,o 8192x8192; k,v 1024x8192; gate,up 28672x8192;
    down 8192x28672) with a seeded retention per tensor drawn from
    U[0.10, 0.50], all seven tensors (seven different k) in one launch; the
    same layer through the fused launch (hh_hctt_decode_lz4_fused_tpb, 10-17
    tiles per block by tensor) bit-identical to it.
"""
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


def decode(L, dtype):
    """One hh_hctt_decode_lz4_batch call over the whole layer; returns the
    device outputs, the LZ4 status codes, the scratch and the tile statuses."""
    Hm = H()
    T = G.torch()
    d_in = G.dev(L["blob"])
    tabs = [G.dev(L[x]) for x in ("in_off", "in_len", "out_off", "out_cap")]
    n = L["in_off"].size
    scratch = T.empty(L["scratch_bytes"], dtype=T.uint8, device="cuda")
    status = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    tdt = {Hm.F32: T.float32, Hm.BF16: T.bfloat16, Hm.F16: T.float16}[dtype]
    outs, tst, desc = [], [], []
    for t in L["tensors"]:
        o = T.empty(t["rows"] * t["cols"], dtype=tdt, device="cuda")
        s = T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda")
        outs.append(o)
        tst.append(s)
        desc.append((scratch.data_ptr() + t["soff"], t["tiles"].size, t["rows"], t["cols"], t["k"], o, s))
    print(f"[layer] {len(desc)} tensors, {n} LZ4 blocks, dtype {dtype}", flush=True)
    G.ctx().hctt_decode_lz4_batch(d_in, d_in.numel(), *tabs[:2], scratch, *tabs[2:], n, status, desc,
                                  dtype=dtype, stream=G.stream())
    G.sync()
    codes = status.cpu().numpy().view(np.int32)[0::8]
    return outs, codes, scratch, tst


def decode_fused(L, dtype):
    """The layer through one hh_hctt_decode_lz4_fused_tpb launch (tensor
    i's blocks hold block_bytes // tile_bytes_i tiles); returns the device
    outputs, the LZ4 status codes and the tile statuses."""
    Hm = H()
    T = G.torch()
    d_in = G.dev(L["blob"])
    in_off, in_len = G.dev(L["in_off"]), G.dev(L["in_len"])
    n = L["in_off"].size
    status = T.zeros(n * 32, dtype=T.uint8, device="cuda")
    tdt = {Hm.F32: T.float32, Hm.BF16: T.bfloat16, Hm.F16: T.float16}[dtype]
    outs, tst, desc, tpb = [], [], [], []
    for t in L["tensors"]:
        o = T.empty(t["rows"] * t["cols"], dtype=tdt, device="cuda")
        s = T.full(((t["rows"] // 64) * (t["cols"] // 64),), -1, dtype=T.int32, device="cuda")
        outs.append(o)
        tst.append(s)
        desc.append((t["rows"], t["cols"], t["k"], o, s))
        tpb.append(max(1, 16384 // Hm.hctt_tile_bytes(t["k"])))
    print(f"[layer] fused: {len(desc)} tensors, {n} LZ4 blocks, tiles per block {tpb}", flush=True)
    rc = G.ctx().hctt_decode_lz4_fused(d_in, d_in.numel(), in_off, in_len, n, status, desc, tpb, dtype=dtype,
                                       stream=G.stream())
    assert rc == Hm.OK
    G.sync()
    codes = status.cpu().numpy().view(np.int32)[0::8]
    return outs, codes, tst


def check_against_oracle(L, outs):
    for t, o in zip(L["tensors"], outs):
        rc, ref = O.hctt_decode_tensor(t["tiles"], t["rows"], t["cols"], t["k"])
        assert rc == O.OK
        got = o.cpu().numpy().reshape(t["rows"], t["cols"])
        rms = float(np.sqrt((ref.astype(np.float64) ** 2).mean()))
        err = float(np.abs(got - ref).max())
        print(f"[layer] {t['name']} {t['rows']}x{t['cols']} k={t['k']}: max|err| = {err / rms:.2e} x RMS",
              flush=True)
        assert err <= TOL * rms, (t["name"], err / rms)
        del ref, got


@pytest.fixture(scope="module")
def llama8b():
    Hm = H()
    k = Hm.hctt_retain_count(0.3)
    assert k == 1228
    return LU.encode_layer(Hm, LU.L8B, [k] * 7, seed=8)


def test_llama3_8b_layer_f32_matches_oracle(llama8b):
    L = llama8b
    assert L["scratch_bytes"] == 218103808 // 4096 * 1204
    assert (L["out_cap"][:-1] == 13 * 1204).any()
    outs, codes, scratch, tst = decode(L, H().F32)
    assert (codes == 0).all()
    # LZ4 output bit-identical to the tile bytes the encoder made
    sc = scratch.cpu().numpy()
    for t in L["tensors"]:
        assert np.array_equal(sc[t["soff"]:t["soff"] + t["tiles"].size], t["tiles"]), t["name"]
    assert all((s.cpu().numpy() == 0).all() for s in tst)
    check_against_oracle(L, outs)


def test_llama3_8b_layer_bf16_is_rne_of_f32(llama8b):
    Hm = H()
    T = G.torch()
    L = llama8b
    f32, codes, _, _ = decode(L, Hm.F32)
    assert (codes == 0).all()
    bf, codes, _, _ = decode(L, Hm.BF16)
    assert (codes == 0).all()
    for t, a, b in zip(L["tensors"], f32, bf):
        # torch's device conversion is round-to-nearest-even (pinned on a
        # sample against the host conversion below)
        assert T.equal(b.view(T.int16), a.to(T.bfloat16).view(T.int16)), t["name"]
    gate = L["tensors"][4]["name"]
    assert gate == "gate"
    a = f32[4].cpu().numpy()
    assert np.array_equal(bf[4].view(T.int16).cpu().numpy().view(np.uint16), G.bf16_bits(a))


def test_llama70b_layer_mixed_retention_matches_oracle():
    Hm = H()
    rng = np.random.default_rng(70)
    rhos = rng.uniform(0.10, 0.50, len(LU.L70B))
    ks = [Hm.hctt_retain_count(float(r)) for r in rhos]
    assert len(set(ks)) == len(ks)
    L = LU.encode_layer(Hm, LU.L70B, ks, seed=71)
    assert L["scratch_bytes"] == sum(r * c // 4096 * Hm.hctt_tile_bytes(k) for (_, r, c), k in zip(LU.L70B, ks))
    outs, codes, scratch, tst = decode(L, Hm.F32)
    assert (codes == 0).all()
    assert all((s.cpu().numpy() == 0).all() for s in tst)
    del scratch
    check_against_oracle(L, outs)
    # the fused launch: the same bits, with no tile bytes in HBM
    T = G.torch()
    fo, fcodes, ftst = decode_fused(L, Hm.F32)
    assert (fcodes == 0).all()
    assert all((s.cpu().numpy() == 0).all() for s in ftst)
    for t, a, b in zip(L["tensors"], outs, fo):
        assert T.equal(a.view(T.int32), b.view(T.int32)), t["name"]
