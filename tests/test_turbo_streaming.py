"""Turbo output files and the progressive loader.

* TurboWriter / TurboReader against the layout of write_output
  (crates/haagenti/src/pipeline/turbo.rs:378-463): u64 header length,
  compact JSON, zstd frame per tensor around the fragment container, XXH3-64
  per fragment; the frames decode with libzstd (pyarrow) and files whose
  frames libzstd wrote at level 1 (as the reference writes them) read back;
* the loader types' own tests (crates/haagenti/src/streaming.rs:416-510)
  and, on the GPU, hh_turbo_tensor_decode and the progressive loader against
  the oracle's reconstruction of the same fragments."""
import json
import struct

import numpy as np
import pytest

import oracle_lib as O
from test_oracle_hct3 import encode, mse, sin_input

TOL = 1e-3


def H():
    import haagenti_amd as h
    return h


def T():
    import haagenti_amd.turbo as t
    return t


def S():
    import haagenti_amd.streaming as s
    return s


def split_container(c):
    """The container split by hand: [(idx, flags, sum, data)]."""
    n = struct.unpack_from("<H", c)[0]
    off, out = 2, []
    for _ in range(n):
        i, fl, s, ln = struct.unpack_from("<HHQI", c, off)
        out.append((i, fl, s, c[off + 16:off + 16 + ln]))
        off += 16 + ln
    assert off == len(c)
    return out


def tensors():
    rng = np.random.default_rng(5)
    x = sin_input(64 * 64, 0.01)
    yield "layers.0.attn.q_proj.weight", [64, 64], encode(x, 64, 64, 4, 0.2)
    y = rng.normal(0, 0.02, 48 * 80).astype(np.float32)
    yield "layers.0.mlp.up_proj.weight", [48, 80], encode(y, 80, 48, 4, 0.3)
    z = rng.normal(0, 1, 300).astype(np.float32)
    yield "norm.weight", [300], encode(z, 300, 1, 2, 0.5)


def test_writer_layout_and_reader_roundtrip(tmp_path):
    pa = pytest.importorskip("pyarrow")
    w = T().TurboWriter()
    ts = list(tensors())
    for name, shape, frags in ts:
        w.add_tensor(name, frags, shape)
    blob = w.to_bytes()
    hl = struct.unpack_from("<Q", blob)[0]
    meta = json.loads(blob[8:8 + hl])
    assert blob[8:8 + hl] == json.dumps(meta, separators=(",", ":")).encode()
    off = 0
    for name, shape, frags in ts:
        m = meta[name]
        assert m["dtype"] == "hct_v3" and m["shape"] == shape and m["data_offsets"][0] == off
        s, e = m["data_offsets"]
        frame = blob[8 + hl + s:8 + hl + e]
        off = e
        size = struct.unpack_from("<Q", frame, 5)[0]       # single-segment frame content size
        c = pa.Codec("zstd").decompress(frame, decompressed_size=size, asbytes=True)
        parts = split_container(c)
        assert [(i, d) for i, _, _, d in parts] == frags
        assert all(fl == 0 and sm == H().xxh3_64(d) for _, fl, sm, d in parts)
    assert 8 + hl + off == len(blob)
    path = tmp_path / "model.hct"
    w.write(path)
    r = T().TurboReader(str(path))
    assert r.tensor_names() == [n for n, _, _ in ts]
    for name, shape, frags in ts:
        assert r.fragments(name) == frags
        assert r.info(name)[1] == shape
    r.close()


def test_reader_takes_libzstd_level1_frames():
    # the reference compresses each container at zstd level 1
    pa = pytest.importorskip("pyarrow")
    ts = list(tensors())
    meta, data = {}, b""
    for name, shape, frags in ts:
        f = pa.Codec("zstd", compression_level=1).compress(H().hct3_container(frags), asbytes=True)
        meta[name] = {"dtype": "hct_v3", "shape": shape, "data_offsets": [len(data), len(data) + len(f)]}
        data += f
    hdr = json.dumps(meta, separators=(",", ":")).encode()
    r = T().TurboReader(struct.pack("<Q", len(hdr)) + hdr + data)
    for name, _, frags in ts:
        assert r.fragments(name) == frags


def test_reader_errors():
    Hm = H()
    name, shape, frags = next(tensors())
    w = T().TurboWriter()
    w.add_tensor(name, frags, shape)
    blob = bytearray(w.to_bytes())
    # a flipped byte inside the last fragment's data: the frame's XXH64 and
    # the fragment's XXH3 both catch it
    bad = bytearray(blob)
    bad[-10] ^= 0x40
    with pytest.raises(Hm.HaagentiError) as e:
        T().TurboReader(bytes(bad)).fragments(name)
    assert e.value.code == Hm.CORRUPTED_DATA
    # a wrong fragment checksum inside an intact frame
    c = bytearray(Hm.hct3_container(frags))
    c[2 + 4] ^= 1
    f = T().zstd_frame_raw(bytes(c))
    hdr = json.dumps({name: {"dtype": "hct_v3", "shape": shape, "data_offsets": [0, len(f)]}}).encode()
    r = T().TurboReader(struct.pack("<Q", len(hdr)) + hdr + f)
    with pytest.raises(Hm.HaagentiError) as e:
        r.fragments(name)
    assert e.value.code == Hm.CHECKSUM_MISMATCH
    assert r.fragments(name, verify=False)[0][1] == frags[0][1]
    with pytest.raises(Hm.HaagentiError):
        T().TurboReader(b"\x10\0\0\0\0\0\0\0{}")
    with pytest.raises(Hm.HaagentiError):
        T().parse_fragment_container(b"\x01\x00" + bytes(10))


def test_dims_follow_process_tensor():
    # turbo.rs:334-343
    assert T().dims([4096, 11008]) == (11008, 4096)
    assert T().dims([300]) == (300, 1)
    assert T().dims([2, 3, 5]) == (5, 6)


def test_load_priority_fraction():
    P = S().LoadPriority
    assert [p.detail_fraction() for p in (P.EssentialsOnly, P.QuickStart, P.Balanced, P.Full)] == [0, 0.15, 0.5, 1]


def test_streaming_tensor_loader_creation_and_status():
    l = S().StreamingTensorLoader("test.weight", 128, 128)
    assert l.name() == "test.weight" and l.dimensions() == (128, 128) and not l.can_reconstruct()
    assert abs(S().StreamingTensorLoader("t", 64, 64).with_mean(0.5).mean_value - 0.5) < 0.01
    st = l.status()
    assert not st.essentials_loaded and st.details_loaded == 0 and not st.complete
    assert l.decoder.quality() == 0.0
    with pytest.raises(H().HaagentiError):
        l.reconstruct()


def test_streaming_model_loader_and_config():
    m = S().StreamingModelLoader(S().LoadPriority.Balanced)
    m.add_tensor(S().StreamingTensorLoader("layer.0.weight", 64, 64))
    m.add_tensor(S().StreamingTensorLoader("layer.1.weight", 64, 64))
    assert m.tensor_count() == 2 and m.ready_count() == 0 and m.progress() == 0.0
    assert m.load_next_round() == 0 and m.is_parallel() and not m.with_parallel(False).is_parallel()
    assert S().StreamingModelLoader(S().LoadPriority.Full).progress() == 1.0
    c = S().ProgressiveLoadConfig()
    assert (c.initial_priority, c.target_priority, c.batch_size) == (S().LoadPriority.EssentialsOnly,
                                                                   S().LoadPriority.Full, 10)
    assert S().ProgressiveLoadConfig.fast_start().batch_size == 20
    assert S().ProgressiveLoadConfig.balanced().initial_priority == S().LoadPriority.QuickStart
    assert S().ProgressiveLoadConfig.high_quality().batch_size == 5


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) or 1.0
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / rms)


@pytest.mark.gpu
def test_turbo_tensor_decode_vs_oracle():
    import gpu_util as G
    Hm = H()
    w = T().TurboWriter()
    ts = list(tensors())
    for name, shape, frags in ts:
        w.add_tensor(name, frags, shape)
    # a container whose fragment 0 is not first decodes the same
    name0, shape0, frags0 = ts[0]
    w.add_tensor("shuffled", [frags0[2], frags0[0], frags0[1], frags0[3]], shape0)
    r = T().TurboReader(w.to_bytes())
    for name, shape, frags in ts + [("shuffled", shape0, frags0)]:
        ref, e, _, _ = O.spectral_reconstruct(frags)
        assert e.kind == O.OK
        got = r.decode_gpu(name, G.ctx(), stream=G.stream())
        G.sync()
        assert tuple(got.shape) == tuple(shape)
        assert rel_err(got.cpu().numpy().ravel(), ref) <= TOL
        b16 = r.decode_gpu(name, G.ctx(), dtype=Hm.BF16)
        assert np.array_equal(b16.view(G.torch().int16).cpu().numpy().ravel().view(np.uint16),
                              G.bf16_bits(got.cpu().numpy().ravel()))


@pytest.mark.gpu
def test_turbo_tensor_decode_errors():
    import gpu_util as G
    Hm = H()
    name, shape, frags = next(tensors())
    c = bytearray(Hm.hct3_container(frags))
    p = 2 + 16 + len(frags[0][1]) + 4        # the checksum of fragment 1
    c[p] ^= 1
    f = T().zstd_frame_raw(bytes(c))
    hdr = json.dumps({name: {"dtype": "hct_v3", "shape": shape, "data_offsets": [0, len(f)]}}).encode()
    r = T().TurboReader(struct.pack("<Q", len(hdr)) + hdr + f)
    with pytest.raises(Hm.HaagentiError) as e:
        r.decode_gpu(name, G.ctx())
    assert e.value.code == Hm.CHECKSUM_MISMATCH and e.value.status.position == 1
    ref = O.spectral_reconstruct(frags)[0]
    assert rel_err(r.decode_gpu(name, G.ctx(), verify=False).cpu().numpy().ravel(), ref) <= TOL
    for blob in [b"\x28\xb5\x2f\xfd\x00\x00", b"\x00\x00", b"\x01"]:
        st = Hm.BlockStatus()
        ww, hh = Hm._u32(0), Hm._u32(0)
        import ctypes as C
        out = G.torch().empty(16, device="cuda")
        rc = Hm.lib().hh_turbo_tensor_decode(G.ctx().handle, blob, len(blob), 1, 0, Hm._addr(out), 16,
                                            C.byref(ww), C.byref(hh), C.byref(st), None)
        assert rc == Hm.CORRUPTED_DATA


@pytest.mark.gpu
def test_streaming_loader_integration():
    # streaming.rs:472-509, plus the reconstruction against the oracle
    import gpu_util as G
    x = sin_input(4096, 0.01)
    mean = float(np.float32(x.sum(dtype=np.float32) / np.float32(4096)))
    frags = H().CompressiveSpectralEncoder(4, 0.70, ctx=G.ctx()).encode_2d(x, 64, 64)
    l = S().StreamingTensorLoader("test", 64, 64, ctx=G.ctx()).with_mean(mean)
    l.add_fragment(frags[0])
    assert l.can_reconstruct() and l.status().essentials_loaded
    assert l.total_details == 1                     # ceil(quality()) as the reference computes it
    for f in frags[1:]:
        l.queue_fragment(f)
    q0 = l.decoder.quality()
    first = l.reconstruct()
    ref0 = O.spectral_reconstruct(frags[:1])[0] + np.float32(mean)
    assert rel_err(first, ref0) <= TOL
    assert l.load_all_pending() == 3
    q1 = l.decoder.quality()
    assert q1 >= q0 and abs(q1 - 1.0) < 1e-6 and l.status().complete
    # LIFO: the last queued detail went in first; the result does not depend on it
    full = l.reconstruct()
    ref = O.spectral_reconstruct(frags)[0] + np.float32(mean)
    assert rel_err(full, ref) <= TOL
    assert mse(x, full - mean) < mse(x, first - mean)


@pytest.mark.gpu
def test_model_loader_rounds_from_file(tmp_path):
    import gpu_util as G
    w = T().TurboWriter()
    ts = list(tensors())
    for name, shape, frags in ts:
        w.add_tensor(name, frags, shape)
    w.write(tmp_path / "m.hct")
    r = T().TurboReader(str(tmp_path / "m.hct"))
    m = S().StreamingModelLoader(S().LoadPriority.Full)
    for name, _, _ in ts:
        m.add_tensor(r.streaming_loader(name, G.ctx()))
    assert m.ready_count() == 3
    # before any detail the decoder does not know the fragment count and
    # reports 1.0 (compressive.rs:720-722); from the first detail on the
    # progress rises to 1.0
    assert m.progress() == 1.0
    seen = []
    while m.load_next_round():
        seen.append(m.progress())
    assert len(seen) == 3 and seen == sorted(seen) and seen[0] < 1.0 and abs(seen[-1] - 1.0) < 1e-6
    for name, _, frags in ts:
        assert rel_err(m.get(name).reconstruct(), O.spectral_reconstruct(frags)[0]) <= TOL
    r.close()


@pytest.mark.gpu
def test_turbo_decode_of_libzstd_level1_frames():
    # the frames the reference writes (zstd level 1, turbo.rs:389-391),
    # decoded by hh_turbo_tensor_decode
    pa = pytest.importorskip("pyarrow")
    import gpu_util as G
    ts = list(tensors())
    meta, data = {}, b""
    for name, shape, frags in ts:
        f = pa.Codec("zstd", compression_level=1).compress(H().hct3_container(frags), asbytes=True)
        meta[name] = {"dtype": "hct_v3", "shape": shape, "data_offsets": [len(data), len(data) + len(f)]}
        data += f
    hdr = json.dumps(meta, separators=(",", ":")).encode()
    r = T().TurboReader(struct.pack("<Q", len(hdr)) + hdr + data)
    for name, shape, frags in ts:
        got = r.decode_gpu(name, G.ctx()).cpu().numpy().ravel()
        assert rel_err(got, O.spectral_reconstruct(frags)[0]) <= TOL
