"""HCT3 whole-tensor spectral decode on the GPU against the oracle.

* hh_hct3_coefficients (GpuDecompressor::reconstruct_coefficients,
  crates/haagenti-cuda/src/decompress.rs:322-427): bit-exact dense
  coefficients, every container edge case the oracle covers;
* hh_hct3_decompress / _device, hh_spectral_reconstruct, hh_idct_2d /
  hh_dct_2d: whole-matrix transforms within 1e-3 x RMS of the oracle's
  restatement of the reference's idct_2d (crates/haagenti-core/src/dct.rs:
  311-337) -- the IDCT tolerance of the decode path; the achieved error is
  ~1e-6 x RMS -- and against the reference's own C decoder where it is
  built; 16-bit outputs are the round-to-nearest-even of the f32 result.

Both whole-matrix routes are covered (the context's HH_OPT_DCT_ROUTE): the
dense split-f16 MFMA products and the FFT route (Makhoul row transforms over
an f32 FFT in LDS, the route the reference takes above 4096,
crates/haagenti-cuda/src/dct_gpu.rs:1081,1404-1412)."""
import contextlib
import struct

import numpy as np
import pytest

import gpu_util as G
import oracle_lib as O
from test_oracle_hct3 import container, encode, mse, random_fragment, sin_input

pytestmark = pytest.mark.gpu
TOL = 1e-3


def H():
    import haagenti_amd as h
    return h


def dec():
    return H().GpuDecompressor(G.ctx())


@contextlib.contextmanager
def route(name):
    G.ctx().set_dct_route(name)
    try:
        yield
    finally:
        G.ctx().set_dct_route("auto")


@pytest.fixture
def dense_route():
    with route("dense"):
        yield


def basis(n, kk):
    s = np.sqrt((1.0 if kk == 0 else 2.0) / n)
    return s * np.cos(np.pi * kk * (2 * np.arange(n) + 1) / (2 * n))


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) or 1.0
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / rms)


@pytest.mark.parametrize("total", [1, 7, 63, 64, 65, 1000, 16383, 16384, 16385, 100003])
def test_coefficients_bit_exact(total):
    rng = np.random.default_rng(total)
    frags = [random_fragment(rng, total, 0.3), random_fragment(rng, total, 0.05),
             random_fragment(rng, total, 0.2, nvals=max(1, total // 20))]
    data = container(frags)
    got = dec().reconstruct_coefficients_gpu(data, total, stream=G.stream()).cpu().numpy()
    rc, ref = O.hct3_coefficients(data, total)
    assert rc == O.OK
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_coefficients_container_edges():
    Hm = H()
    rng = np.random.default_rng(11)
    total = 300
    bm, vals, _ = random_fragment(rng, total, 0.5)
    ok = container([(bm, vals, None)])
    cases = [ok, struct.pack("<H", 2) + ok[2:] + b"\0" * 5,
             struct.pack("<H", 3) + struct.pack("<HHQI", 0, 0, 0, 3) + b"abc"
             + struct.pack("<HHQI", 1, 0, 0, 10) + bytes(10) + ok[2:],
             container([(bm, vals[:7], 99)]), struct.pack("<H", 0)]
    for data in cases:
        got = dec().reconstruct_coefficients_gpu(data, total).cpu().numpy()
        assert np.array_equal(got, O.hct3_coefficients(data, total)[1])
    for bad in [b"\x01", ok[:-1]]:
        with pytest.raises(Hm.HaagentiError) as e:
            dec().reconstruct_coefficients_gpu(bad, total)
        assert e.value.code == Hm.INVALID_ARGUMENT
        assert O.hct3_coefficients(bad, total)[0] == O.INVALID_DATA
    # zstd magic that is not a zstd stream: parsed as a raw container, as
    # try_zstd_decompress falls back (decompress.rs:306-316)
    fake = b"\x28\xb5\x2f\xfd" + ok
    rc, _ = O.hct3_coefficients(fake, total)
    if rc == O.OK:
        got = dec().reconstruct_coefficients_gpu(fake, total).cpu().numpy()
        assert np.array_equal(got, O.hct3_coefficients(fake, total)[1])
    else:
        with pytest.raises(Hm.HaagentiError) as e:
            dec().decompress_to_gpu(fake, [total])
        assert e.value.code == Hm.INVALID_ARGUMENT


def test_zstd_wrapped_container():
    # the turbo wrapper: zstd level 1 over the container (turbo.rs:389-391)
    pa = pytest.importorskip("pyarrow")
    T = G.torch()
    rng = np.random.default_rng(13)
    shape = (96, 160)
    total = 96 * 160
    data = container([random_fragment(rng, total, 0.2), random_fragment(rng, total, 0.1)])
    wrapped = pa.Codec("zstd", compression_level=1).compress(data, asbytes=True)
    assert wrapped[:4] == b"\x28\xb5\x2f\xfd"
    raw = dec().decompress_to_gpu(data, shape).cpu().numpy()
    got = dec().decompress_to_gpu(wrapped, shape).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), raw.view(np.uint32))
    out = T.empty(total, dtype=T.float32, device="cuda")
    dec().decompress_device(wrapped, G.dev(np.frombuffer(wrapped, np.uint8)), shape, out)
    G.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), raw.view(np.uint32))


@pytest.mark.parametrize("shape", [(64, 64), (37, 53), (1, 1000), (1000,), (3, 5, 17), (256, 512), (96, 4)])
def test_decompress_f32_vs_oracle(shape):
    rng = np.random.default_rng(sum(shape))
    total = int(np.prod(shape))
    data = container([random_fragment(rng, total, 0.25), random_fragment(rng, total, 0.05)])
    got = dec().decompress_to_gpu(data, shape, stream=G.stream()).cpu().numpy()
    rc, ref = O.hct3_decode(data, shape)
    assert rc == O.OK
    err = rel_err(got, ref)
    print(f"shape {shape}: max|gpu - oracle| = {err:.2e} x RMS")
    assert err <= TOL
    if O.ref_available() and total <= 64 * 64:
        w = shape[-1]
        c = O.ref_hct_decode(data, total // w, w)
        assert rel_err(got, c.ravel()) <= TOL


def test_decompress_16bit_outputs_and_device_variant():
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(12)
    shape = (128, 192)
    total = 128 * 192
    data = container([random_fragment(rng, total, 0.3)])
    f32 = dec().decompress_to_gpu(data, shape).cpu().numpy()
    b16 = dec().decompress_to_gpu(data, shape, dtype=Hm.BF16).view(T.int16).cpu().numpy().view(np.uint16)
    h16 = dec().decompress_to_gpu(data, shape, dtype=Hm.F16).view(T.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(b16, G.bf16_bits(f32))
    assert np.array_equal(h16, G.f16_bits(f32))
    d_data = G.dev(np.frombuffer(data, np.uint8))
    out = T.empty(total, dtype=T.float32, device="cuda")
    dec().decompress_device(data, d_data, shape, out, stream=G.stream())
    G.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), f32.view(np.uint32))


@pytest.mark.parametrize("way", ["dense", "fft"])
@pytest.mark.parametrize("rows,cols", [(64, 64), (1, 77), (77, 1), (37, 53), (200, 120), (512, 512), (1024, 512),
                                       (512, 1536), (192, 2048)])
def test_idct_dct_2d(rows, cols, way):
    # against the f64 closed form; "fft" takes the FFT route where both sides
    # allow it (multiples of 64 whose halves factor into 2, 3, 5, 7) and the
    # dense route for the others
    T = G.torch()
    rng = np.random.default_rng(rows + 7 * cols)
    c = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    d_c = T.from_numpy(c).cuda()
    x = T.empty_like(d_c)
    y = T.empty_like(d_c)
    with route(way):
        G.ctx().idct_2d(d_c, rows, cols, x, stream=G.stream())
        # forward, and the round trip
        G.ctx().dct_2d(x, rows, cols, y, stream=G.stream())
        G.sync()
    x64 = np.zeros((rows, cols))
    O.lib().hho_idct_2d_f64(O._p(c.astype(np.float64)), O._p(x64), cols, rows)
    assert rel_err(x.cpu().numpy(), x64) <= 1e-5
    assert rel_err(y.cpu().numpy(), c) <= 1e-5


@pytest.mark.usefixtures("dense_route")
@pytest.mark.parametrize("rows,cols,k,l", [(512, 1024, 5, 30), (1024, 512, 0, 1), (512, 512, 511, 256)])
def test_idct_even_odd_split_single_coefficient(rows, cols, k, l):
    # sides that are multiples of 512 take the even / odd split of the bases:
    # one coefficient of either frequency parity per axis lands in the right
    # rows (i and n - 1 - i) with the right sign
    T = G.torch()
    c = np.zeros((rows, cols), np.float32)
    c[k, l] = 1.0
    x = T.empty(rows, cols, dtype=T.float32, device="cuda")
    G.ctx().idct_2d(T.from_numpy(c).cuda(), rows, cols, x)
    ref = np.outer(basis(rows, k), basis(cols, l))
    assert np.abs(x.cpu().numpy() - ref).max() <= 1e-6


# lengths whose halves run radix 8, 4 (64, 192, 1536, 320, 448, 1344), 2
# (2048: three radix-8 passes and one radix-2 with four butterflies per
# thread, the widest variant), 3 (192, 1536, 1344), 5 (320, 640), 7 (448,
# 896, 1344)
@pytest.mark.parametrize("rows,cols", [(64, 192), (320, 448), (1536, 640), (896, 1344), (2048, 128)])
def test_fft_route_single_coefficient_closed_form(rows, cols):
    # C = e_k e_l^T inverts to the outer product of two basis rows, and the
    # forward transform of that product is e_k e_l^T again; k, l include 0,
    # n/2 and n-1, which the real-to-complex packing pairs specially
    T = G.torch()
    with route("fft"):
        for k, l in [(0, 0), (rows // 2, 1), (rows - 1, cols // 2), (7, cols - 1), (rows // 4 + 3, cols // 4)]:
            c = np.zeros((rows, cols), np.float32)
            c[k, l] = 1.0
            x = T.empty(rows, cols, dtype=T.float32, device="cuda")
            G.ctx().idct_2d(T.from_numpy(c).cuda(), rows, cols, x)
            ref = np.outer(basis(rows, k), basis(cols, l))
            assert np.abs(x.cpu().numpy() - ref).max() <= 1e-6, (k, l)
            y = T.empty_like(x)
            G.ctx().dct_2d(T.from_numpy(ref.astype(np.float32)).cuda(), rows, cols, y)
            assert np.abs(y.cpu().numpy() - c).max() <= 1e-5, (k, l)


def test_fft_route_matches_dense_route_4096():
    # one 4096 x 4096 HCT3 tensor decoded on both routes (f32 within
    # 1e-5 x RMS of each other); the FFT route's bf16 and f16 outputs are the
    # rounding of its f32 output, and the device-resident entry gives the
    # same bits
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(4097)
    shape = (4096, 4096)
    total = 4096 * 4096
    data = container([random_fragment(rng, total, 0.2), random_fragment(rng, total, 0.02)])
    with route("dense"):
        dense = dec().decompress_to_gpu(data, shape, stream=G.stream()).cpu().numpy()
    with route("fft"):
        got = dec().decompress_to_gpu(data, shape, stream=G.stream()).cpu().numpy()
        b16 = dec().decompress_to_gpu(data, shape, dtype=Hm.BF16).view(T.int16).cpu().numpy().view(np.uint16)
        h16 = dec().decompress_to_gpu(data, shape, dtype=Hm.F16).view(T.int16).cpu().numpy().view(np.uint16)
        out = T.empty(total, dtype=T.float32, device="cuda")
        dec().decompress_device(data, G.dev(np.frombuffer(data, np.uint8)), shape, out, stream=G.stream())
        G.sync()
    err = rel_err(got, dense)
    print(f"[hct3] 4096 x 4096: max|fft - dense| = {err:.2e} x RMS", flush=True)
    assert err <= 1e-5
    assert np.array_equal(b16, G.bf16_bits(got))
    assert np.array_equal(h16, G.f16_bits(got))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("odd", [False, True])
def test_fft_route_fragments_scattered_in_the_first_pass(odd):
    # on the FFT route the first row pass builds each row from the fragments
    # in LDS: three fragments, the second overwriting part of the first, the
    # third running out of values; values 2-byte aligned, or read bytewise
    # when the container sits at an odd device address -- against the oracle
    # and the dense route
    T = G.torch()
    rng = np.random.default_rng(777 + int(odd))
    shape = (1024, 1536)
    total = shape[0] * shape[1]
    bm2, v2, _ = random_fragment(rng, total, 0.02)
    data = container([random_fragment(rng, total, 0.2), random_fragment(rng, total, 0.05),
                      (bm2, v2[: v2.size // 2], None)])
    rc, ref = O.hct3_decode(data, shape)
    assert rc == O.OK
    with route("dense"):
        dense = dec().decompress_to_gpu(data, shape).cpu().numpy()
    raw = np.frombuffer(data, np.uint8)
    buf = np.zeros(raw.size + 1, np.uint8)
    buf[int(odd):int(odd) + raw.size] = raw
    d_buf = G.dev(buf)
    out = T.empty(total, dtype=T.float32, device="cuda")
    with route("fft"):
        dec().decompress_device(data, d_buf[int(odd):], shape, out, stream=G.stream())
        G.sync()
    got = out.cpu().numpy()
    e_ref, e_dense = rel_err(got, ref), rel_err(got, dense)
    print(f"[hct3] fused scatter (odd={odd}): max|fft - oracle| = {e_ref:.2e}, |fft - dense| = {e_dense:.2e} x RMS")
    assert e_ref <= 1e-5 and e_dense <= 2e-5


@pytest.mark.usefixtures("dense_route")
def test_decompress_even_odd_split_vs_oracle_and_16bit():
    # a 1024 x 512 HCT3 tensor: the split inverse against the oracle, and its
    # bf16 / f16 outputs the rounding of its f32 output
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(1536)
    shape = (1024, 512)
    total = 1024 * 512
    data = container([random_fragment(rng, total, 0.25), random_fragment(rng, total, 0.05)])
    got = dec().decompress_to_gpu(data, shape, stream=G.stream()).cpu().numpy()
    rc, ref = O.hct3_decode(data, shape)
    assert rc == O.OK
    err = rel_err(got, ref)
    print(f"shape {shape}: max|gpu - oracle| = {err:.2e} x RMS")
    assert err <= TOL
    b16 = dec().decompress_to_gpu(data, shape, dtype=Hm.BF16).view(T.int16).cpu().numpy().view(np.uint16)
    h16 = dec().decompress_to_gpu(data, shape, dtype=Hm.F16).view(T.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(b16, G.bf16_bits(got))
    assert np.array_equal(h16, G.f16_bits(got))


def _direct_vs_dense(data, shape):
    # the direct plane scatter (host-staged and device-resident entries)
    # against the oracle and against the dense route (hh_hct3_coefficients,
    # then hh_idct_2d); returns the f32 output and the two differences
    T = G.torch()
    total = shape[0] * shape[1]
    rc, ref = O.hct3_decode(data, shape)
    assert rc == O.OK
    got = dec().decompress_to_gpu(data, shape, stream=G.stream()).cpu().numpy()
    out = T.empty(total, dtype=T.float32, device="cuda")
    dec().decompress_device(data, G.dev(np.frombuffer(data, np.uint8)), shape, out, stream=G.stream())
    G.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), got.view(np.uint32))
    coef = dec().reconstruct_coefficients_gpu(data, total, stream=G.stream())
    x = T.empty(total, dtype=T.float32, device="cuda")
    G.ctx().idct_2d(coef, shape[0], shape[1], x, stream=G.stream())
    G.sync()
    e_ref, e_dense = rel_err(got, ref), rel_err(got, x.cpu().numpy())
    print(f"shape {shape}: max|gpu - oracle| = {e_ref:.2e}, max|direct - dense| = {e_dense:.2e} x RMS")
    return got, e_ref, e_dense


@pytest.mark.usefixtures("dense_route")
def test_decompress_direct_plane_scatter_matches_dense_route():
    # sides that are multiples of 512: the fragments' values are scattered
    # straight into the split transform's operand plane, scaled by a power of
    # two from the largest value of any fragment; with the largest value in
    # the final matrix that is the dense route's scale
    Hm = H()
    T = G.torch()
    rng = np.random.default_rng(2048)
    shape = (512, 1024)
    total = 512 * 1024
    bm2, v2, _ = random_fragment(rng, total, 0.02)
    data = container([random_fragment(rng, total, 0.2), random_fragment(rng, total, 0.05),
                      (bm2, v2[: v2.size // 2], None)])    # the third runs out of values
    got, e_ref, e_dense = _direct_vs_dense(data, shape)
    assert e_ref <= 1e-5 and e_dense <= 1e-6
    b16 = dec().decompress_to_gpu(data, shape, dtype=Hm.BF16).view(T.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(b16, G.bf16_bits(got))


@pytest.mark.usefixtures("dense_route")
def test_decompress_direct_plane_scatter_overwritten_maximum():
    # the second fragment overwrites part of the first, including its largest
    # value (400, against values of ~0.05): the scale comes from a value the
    # final matrix no longer holds (2^11 smaller than the dense route's), and
    # the error stays at the 1e-6 level
    rng = np.random.default_rng(4096)
    shape = (1024, 512)
    total = 1024 * 512
    bm0, v0, _ = random_fragment(rng, total, 0.2)
    bits0 = np.unpackbits(np.frombuffer(bm0, np.uint8), bitorder="little")[:total].astype(bool)
    v0 = v0.copy()
    v0[0] = np.float16(400.0)
    bits1 = rng.random(total) < 0.05
    bits1[int(np.flatnonzero(bits0)[0])] = True
    v1 = rng.normal(0, 0.05, int(bits1.sum())).astype(np.float16)
    bm1 = np.packbits(bits1.astype(np.uint8), bitorder="little").tobytes()
    data = container([(bm0, v0, None), (bm1, v1, None)])
    _, e_ref, e_dense = _direct_vs_dense(data, shape)
    assert e_ref <= 1e-5 and e_dense <= 1e-5


def test_idct_single_coefficient_closed_form():
    # C = e_k e_l^T  ->  X[i][j] = B_h[k][i] B_w[l][j]
    T = G.torch()
    rows, cols, k, l = 48, 80, 5, 31
    c = np.zeros((rows, cols), np.float32)
    c[k, l] = 1.0
    x = T.empty(rows, cols, dtype=T.float32, device="cuda")
    G.ctx().idct_2d(T.from_numpy(c).cuda(), rows, cols, x)
    ref = np.outer(basis(rows, k), basis(cols, l))
    assert np.abs(x.cpu().numpy() - ref).max() <= 1e-6


def test_spectral_reconstruct_vs_oracle():
    Hm = H()
    x = sin_input(4096, 0.01)
    for w, h, nf, r in [(64, 64, 8, 0.1), (128, 32, 4, 0.3), (4096, 1, 2, 0.2)]:
        frags = encode(x[:w * h], w, h, nf, r)
        for subset in (frags[:1], frags[:max(1, nf // 2)], frags):
            d = Hm.CompressiveSpectralDecoder(G.ctx())
            d.add_essentials(subset[0])
            for f in subset[1:]:
                d.add_detail(f)
            got = d.reconstruct()
            ref, e, _, _ = O.spectral_reconstruct(subset)
            assert e.kind == O.OK
            assert rel_err(got, ref) <= TOL


def test_spectral_reconstruct_errors_match_oracle():
    Hm = H()
    x = sin_input(256, 0.1)
    frags = encode(x, 16, 16, 4, 0.3)
    f0 = frags[0][1]
    g = bytearray(f0)
    g[24] ^= 1
    bad_cases = [[(0, f0[:20])], [(0, f0[:40])], [(0, bytes(g))] + frags[1:], [(0, f0[:-1])],
                 [frags[0], (1, b"\x01\x00")]]
    for case in bad_cases:
        _, e, _, _ = O.spectral_reconstruct(case, 256)
        with pytest.raises(Hm.HaagentiError) as ex:
            d = Hm.CompressiveSpectralDecoder(G.ctx())
            d.add_essentials(case[0])
            for f in case[1:]:
                d.add_detail(f)
            d.reconstruct()
        assert ex.value.code == e.kind == Hm.CORRUPTED_DATA
        assert ex.value.status.detail == e.sub


def test_encoder_gpu_dct_end_to_end():
    # CompressiveSpectralEncoder.encode_2d with the GPU forward DCT, decoded
    # on the GPU: the reference's own bounds (compressive.rs:777-816, 930-962)
    Hm = H()
    for n, side, step, ret, bound in [(256, 16, 0.1, 1.0, 1e-4), (256, 16, 0.1, 0.2, 0.5),
                                      (1024, 32, 0.01, 0.10, 0.5), (1024, 32, 0.01, 0.30, 0.2)]:
        x = sin_input(n, step)
        frags = Hm.CompressiveSpectralEncoder(4, ret, ctx=G.ctx()).encode_2d(x, side, side)
        d = Hm.CompressiveSpectralDecoder(G.ctx())
        d.add_essentials(frags[0])
        for f in frags[1:]:
            d.add_detail(f)
        assert mse(x, d.reconstruct()) < bound
    # a 2048 x 2048 N(0, 0.02) tensor at full retention: decode(encode(w))
    # differs from w only by the f16 rounding of the coefficients
    T = G.torch()
    w = T.randn(2048, 2048, device="cuda") * 0.02
    c = T.empty_like(w)
    G.ctx().dct_2d(w, 2048, 2048, c)
    frags = Hm.CompressiveSpectralEncoder(1, 1.0).with_essential_ratio(1.0).encode_2d_from_dct(
        c.cpu().numpy(), 2048, 2048)
    d = Hm.CompressiveSpectralDecoder(G.ctx())
    d.add_essentials(frags[0])
    back = d.reconstruct_gpu()
    diff = back.cpu().numpy().astype(np.float64) - w.cpu().numpy().ravel()
    assert np.sqrt(np.mean(diff ** 2)) <= 1e-3 * 0.02


def hct2_from_hct3(frags, rng):
    """The same fragments in the f32 layout ("HCT2", compressive.rs:23,
    470-500), values perturbed off the f16 grid so that the inverse DCT
    takes the split path of arbitrary f32 input."""
    f0 = frags[0][1]
    magic, w, h, keep, ess, dpf = struct.unpack_from("<6I", f0)
    bm = (w * h + 7) // 8
    v0 = np.frombuffer(f0[24 + bm:24 + bm + 2 * ess], np.float16).astype(np.float32)
    v0 = (v0 * (1 + rng.normal(0, 1e-3, v0.size))).astype(np.float32)
    out = [(0, struct.pack("<6I", 0x48435432, w, h, keep, ess, dpf) + f0[24:24 + bm] + v0.tobytes())]
    for idx, d in frags[1:]:
        fi, tot, cnt = struct.unpack_from("<HHI", d)
        v = np.frombuffer(d[8:8 + 2 * cnt], np.float16).astype(np.float32)
        v = (v * (1 + rng.normal(0, 1e-3, v.size))).astype(np.float32)
        out.append((idx, struct.pack("<HHI", fi, tot, cnt) + v.tobytes()))
    return out


def test_hct2_f32_fragments_vs_oracle():
    Hm = H()
    rng = np.random.default_rng(21)
    x = sin_input(96 * 160, 0.003)
    for w, h, nf, r in [(160, 96, 4, 0.3), (64, 64, 2, 1.0)]:
        frags = hct2_from_hct3(encode(x[:w * h], w, h, nf, r), rng)
        d = Hm.CompressiveSpectralDecoder(G.ctx())
        d.add_essentials(frags[0])
        for f in frags[1:]:
            d.add_detail(f)
        got = d.reconstruct()
        ref, e, ww, hh = O.spectral_reconstruct(frags)
        assert e.kind == O.OK and (ww, hh) == (w, h)
        assert rel_err(got, ref) <= TOL


def test_decompress_batch_pipelined_matches_decompress():
    # decompress.rs:228-279: same results as one tensor at a time, with the
    # phase statistics the reference reports
    rng = np.random.default_rng(23)
    shapes = [(64, 96), (40, 40), (1, 500)]
    items = []
    for shp in shapes:
        total = int(np.prod(shp))
        items.append((container([random_fragment(rng, total, 0.3)]), shp))
    d = dec()
    outs, stats = d.decompress_batch_pipelined(items)
    assert stats["num_tensors"] == 3 and stats["total_output_bytes"] == 4 * sum(int(np.prod(s)) for s in shapes)
    assert stats["total_input_bytes"] == sum(len(c) for c, _ in items)
    assert stats["total_time_ms"] >= stats["parse_time_ms"] >= 0 and stats["idct_time_ms"] >= 0
    for (c, shp), o in zip(items, outs):
        assert rel_err(o, dec().decompress(c, shp)) <= 1e-5
        assert rel_err(o, O.hct3_decode(c, shp)[1]) <= TOL


def _real_size(rows, cols, seed, way="auto"):
    # one fragment at the turbo pipeline's 20 % retention: the GPU decode
    # (the FFT route at these sizes by default; "dense": direct plane
    # scatter + even / odd split products) against the oracle's bit-exact
    # scatter and f32 idct_2d (the same 1-D transforms as hct3_decode, run on
    # every host thread)
    rng = np.random.default_rng(seed)
    total = rows * cols
    data = container([random_fragment(rng, total, 0.2)])
    print(f"[hct3] {rows} x {cols} ({way}): {len(data)} container bytes", flush=True)
    with route(way):
        got = dec().decompress_to_gpu(data, (rows, cols), stream=G.stream()).cpu().numpy()
    rc, coef = O.hct3_coefficients(data, total)
    assert rc == O.OK
    ref = O.idct_2d_mt(coef.reshape(rows, cols)).ravel()
    del coef
    err = rel_err(got, ref)
    print(f"[hct3] {rows} x {cols}: max|gpu - oracle| = {err:.2e} x RMS", flush=True)
    assert err <= TOL
    return data, got


@pytest.mark.parametrize("rows,cols,way", [(4096, 4096, "dense"), (4096, 4096, "auto"), (8192, 8192, "dense"),
                                           (8192, 8192, "auto")])
def test_decompress_real_sizes_vs_oracle(rows, cols, way):
    data, got = _real_size(rows, cols, seed=rows // 64, way=way)
    if rows == 8192:
        T = G.torch()
        with route(way):
            b16 = dec().decompress_to_gpu(data, (rows, cols), dtype=H().BF16).view(T.int16).cpu().numpy()
        assert np.array_equal(b16.view(np.uint16), G.bf16_bits(got))


def test_decompress_llama70b_mlp_tensor_vs_oracle():
    # a 28672 x 8192 tensor (the Llama-70B gate / up projection's shape)
    _real_size(28672, 8192, seed=28672)
