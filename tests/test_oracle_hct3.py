"""Oracle HCT3 whole-tensor spectral decode and the host-side producer.

Pins:
  * the coefficient scatter of the fragment container
    (crates/haagenti-cuda/src/decompress.rs:322-427) bit-exactly against the
    reference's own C decoder (ref/c/hct_decoder.h, built into oracle/_ref):
    hct_decode(data) must equal hct_idct_2d applied to the oracle's
    coefficient matrix, bit for bit, since both run the same C transform;
  * the oracle's whole-matrix transform against the f64 closed form;
  * CompressiveSpectralEncoder / Decoder (crates/haagenti/src/compressive.rs)
    against each other and the reference's own MSE bounds
    (compressive.rs:777-980), its byte layout, and the product's host encoder
    (hh_spectral_encode_from_dct) byte for byte;
  * half::f16::from_f32 (IEEE round to nearest even) against numpy."""
import struct

import numpy as np
import pytest

import oracle_lib as O


def container(frags):
    """HCT V3 fragment container: [u16 n] + {u16 idx, u16 flags, u64 sum,
    u32 len, [u32 count][bitmap][f16 values]} per fragment."""
    out = struct.pack("<H", len(frags))
    for i, (bm, vals, cnt) in enumerate(frags):
        v = np.ascontiguousarray(vals, dtype=np.float16)
        data = struct.pack("<I", v.size if cnt is None else cnt) + bytes(bm) + v.tobytes()
        out += struct.pack("<HHQI", i, 0, 0, len(data)) + data
    return out


def random_fragment(rng, total, density, nvals=None, scale=0.05):
    bits = rng.random(total) < density
    bm = np.packbits(bits.astype(np.uint8), bitorder="little").tobytes()
    n = int(bits.sum()) if nvals is None else nvals
    vals = rng.normal(0, scale, n).astype(np.float16)
    return bm, vals, None


def test_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    # every f16 value, and every midpoint between neighbours (ties go to even)
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    mids = ((f[:-1].astype(np.float64) + f[1:].astype(np.float64)) / 2).astype(np.float32)
    v = np.concatenate([f, -f, mids, -mids, rng.normal(0, 1, 5000).astype(np.float32),
                        np.array([65504, 65519, 65520, 1e6, np.inf, -np.inf, 1e-9, 5.96e-8], np.float32)])
    got = np.array([O.f32_to_f16_rne(x) for x in v], np.uint16)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    assert (got == ref).all()


@pytest.mark.skipif(not O.ref_available(), reason="reference C decoder not built")
@pytest.mark.parametrize("rows,cols", [(8, 8), (16, 48), (37, 53), (1, 100), (64, 64)])
def test_hct3_scatter_matches_reference_c_decoder(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    total = rows * cols
    frags = [random_fragment(rng, total, 0.2), random_fragment(rng, total, 0.1)]
    data = container(frags)
    rc, dense = O.hct3_coefficients(data, total)
    assert rc == O.OK
    ref = O.ref_hct_decode(data, rows, cols)
    mine = O.ref_idct_2d(dense.reshape(rows, cols))
    assert np.array_equal(ref.view(np.uint32), mine.view(np.uint32))
    # later fragments overwrite earlier ones at their set bits
    bm1 = np.unpackbits(np.frombuffer(frags[1][0], np.uint8), bitorder="little")[:total].astype(bool)
    assert np.array_equal(dense[bm1], frags[1][1].astype(np.float32))


def test_hct3_decode_transform_vs_f64():
    rng = np.random.default_rng(7)
    for shape in [(24, 40), (64, 64), (3, 5, 17), (200,)]:
        total = int(np.prod(shape))
        data = container([random_fragment(rng, total, 0.3)])
        rc, out = O.hct3_decode(data, shape)
        assert rc == O.OK
        _, dense = O.hct3_coefficients(data, total)
        w = shape[-1]
        h = total // w
        d64 = dense.astype(np.float64).reshape(h, w)
        x64 = np.zeros_like(d64)
        O.lib().hho_idct_2d_f64(O._p(d64), O._p(x64), w, h)
        rms = np.sqrt(np.mean(x64 ** 2))
        assert np.abs(out.reshape(h, w) - x64).max() <= 1e-4 * rms  # f32 FFT-path rounding


def test_hct3_container_edge_semantics():
    rng = np.random.default_rng(8)
    total = 100
    bm, vals, _ = random_fragment(rng, total, 0.5)
    ok = container([(bm, vals, None)])
    # shorter than 2 bytes: InvalidData (decompress.rs:324-326)
    assert O.hct3_coefficients(b"\x01", total)[0] == O.INVALID_DATA
    # a fragment extending past the end: InvalidData (:362-367)
    assert O.hct3_coefficients(ok[:-1], total)[0] == O.INVALID_DATA
    # a truncated fragment header ends the scan without error (:335-337)
    rc, d = O.hct3_coefficients(struct.pack("<H", 2) + ok[2:] + b"\x00" * 5, total)
    assert rc == O.OK and np.array_equal(d, O.hct3_coefficients(ok, total)[1])
    # fragments shorter than 4 bytes or than their bitmap are skipped (:373-383)
    short = struct.pack("<H", 3) + struct.pack("<HHQI", 0, 0, 0, 3) + b"abc" + \
        struct.pack("<HHQI", 1, 0, 0, 10) + bytes(10) + ok[2:]
    rc, d = O.hct3_coefficients(short, total)
    assert rc == O.OK and np.array_equal(d, O.hct3_coefficients(ok, total)[1])
    # fewer values than set bits: the first set bits take them, in order
    few = vals[:7]
    rc, d = O.hct3_coefficients(container([(bm, few, 99)]), total)
    set_pos = np.flatnonzero(np.unpackbits(np.frombuffer(bm, np.uint8), bitorder="little")[:total])
    assert rc == O.OK
    assert np.array_equal(d[set_pos[:7]], few.astype(np.float32)) and (d[set_pos[7:]] == 0).all()
    # no fragments: all zeros
    rc, d = O.hct3_coefficients(struct.pack("<H", 0), total)
    assert rc == O.OK and not d.any()


def sin_input(n, step):
    return np.sin(np.arange(n, dtype=np.float32) * np.float32(step)).astype(np.float32)


def encode(x, width, height, nfrag, retention, essential_ratio=0.2):
    """encode_2d (compressive.rs:129-238): dct_2d (dct.rs:282-308), then the
    retention and fragment layout."""
    x = np.ascontiguousarray(x, np.float32)
    c = np.zeros(width * height, np.float32)
    O.lib().hho_dct_2d(O._p(x), O._p(c), width, height)
    return O.spectral_encode_from_dct(c, width, height, nfrag, retention, essential_ratio)


def mse(a, b):
    return float(np.mean((np.asarray(a, np.float64) - np.asarray(b, np.float64)) ** 2))


@pytest.mark.parametrize("n,side,step,nfrag,ret,bound", [
    (256, 16, 0.1, 4, 1.0, 1e-4),    # compressive.rs:777-795
    (256, 16, 0.1, 4, 0.2, 0.5),     # :797-816
    (1024, 32, 0.01, 4, 0.05, 1.0),  # :911-928
    (1024, 32, 0.01, 4, 0.10, 0.5),  # :930-945
    (1024, 32, 0.01, 4, 0.30, 0.2),  # :947-962
])
def test_spectral_roundtrip_reference_bounds(n, side, step, nfrag, ret, bound):
    x = sin_input(n, step)
    frags = encode(x, side, side, nfrag, ret)
    out, e, w, h = O.spectral_reconstruct(frags)
    assert e.kind == O.OK and (w, h) == (side, side)
    assert mse(x, out) < bound


def test_spectral_progressive_and_layout():
    # compressive.rs:848-909: more fragments, lower error
    x = sin_input(256, 0.1)
    frags = encode(x, 16, 16, 8, 0.3)
    e_ess = mse(x, O.spectral_reconstruct(frags[:1])[0])
    e_half = mse(x, O.spectral_reconstruct(frags[:4])[0])
    e_all = mse(x, O.spectral_reconstruct(frags)[0])
    assert e_all <= e_half <= e_ess
    # layout (compressive.rs:174-236)
    f0 = frags[0][1]
    magic, w, h, keep, ess, dpf = struct.unpack_from("<6I", f0)
    assert magic == 0x48435433 and (w, h) == (16, 16)
    assert keep == int(np.float32(256) * np.float32(0.3)) and ess == int(np.float32(keep) * np.float32(0.2))
    assert dpf == -(-(keep - ess) // 7)
    bits = np.unpackbits(np.frombuffer(f0[24:24 + 32], np.uint8), bitorder="little")
    assert bits.sum() == keep and len(f0) == 24 + 32 + 2 * ess
    for f, d in frags[1:]:
        fi, tot, cnt = struct.unpack_from("<HHI", d)
        assert (fi, tot) == (f, 8) and len(d) == 8 + 2 * cnt


def test_spectral_storage_reduction():
    # compressive.rs:818-846
    x = sin_input(4096, 0.01)
    frags = encode(x, 64, 64, 8, 0.1)
    total = sum(len(d) for _, d in frags)
    assert x.nbytes / total > 1.5


def test_product_host_encoder_matches_oracle():
    import haagenti_amd as H
    rng = np.random.default_rng(9)
    cases = [(rng.normal(0, 1, 64 * 48).astype(np.float32), 64, 48, 5, 0.25, 0.2),
             (rng.normal(0, 1, 1000).astype(np.float32), 1000, 1, 1, 0.1, 1.0),
             # many tied magnitudes: the stable order decides
             ((rng.integers(-3, 4, 40 * 40) * 0.5).astype(np.float32), 40, 40, 3, 0.3, 0.5),
             (rng.normal(0, 1e-6, 77 * 13).astype(np.float32), 77, 13, 2, 0.05, 0.05)]
    for c, w, h, nf, r, er in cases:
        mine = H.CompressiveSpectralEncoder(nf, r).with_essential_ratio(er).encode_2d_from_dct(c, w, h)
        ref = O.spectral_encode_from_dct(c, w, h, nf, r, er)
        assert mine == ref
        size = H.lib().hh_spectral_encoded_size(w, h, nf, r, er, None, None)
        assert size == sum(len(d) for _, d in ref)


def test_spectral_decoder_errors():
    x = sin_input(256, 0.1)
    frags = encode(x, 16, 16, 4, 0.3)
    f0 = bytearray(frags[0][1])
    # fragment 0 too short / truncated bitmap (:446-448, :614-616)
    out, e, _, _ = O.spectral_reconstruct([(0, bytes(f0[:20]))], 256)
    assert e.kind == O.CORRUPTED and e.sub == 5
    out, e, _, _ = O.spectral_reconstruct([(0, bytes(f0[:40]))], 256)
    assert e.kind == O.CORRUPTED and e.sub == 5
    # bitmap count mismatch (:630-636)
    g = bytearray(f0)
    g[24] ^= 0x01
    assert O.spectral_reconstruct([(0, bytes(g))] + frags[1:], 256)[1].sub == O.CORRUPT_BITMAP_COUNT
    # truncated essentials (:641-644)
    assert O.spectral_reconstruct([(0, bytes(f0[:-1]))], 256)[1].sub == 5
    # short detail fragment (:667-669)
    assert O.spectral_reconstruct([frags[0], (1, b"\x01\x00")], 256)[1].sub == 5
    # V1 (explicit indices) is not decoded here
    v1 = bytearray(f0)
    v1[0:4] = b"\x00\x00\x00\x00"
    assert O.spectral_reconstruct([(0, bytes(v1))], 256)[1].kind == O.UNSUPPORTED
    # a detail fragment given first
    assert O.spectral_reconstruct([frags[1]], 256)[1].sub == O.CORRUPT_HEADER
