"""Turbo pipeline output files (crates/haagenti/src/pipeline/turbo.rs:315-463).

Layout (write_output, :421-463): [u64 LE header length][compact JSON
{name: {"dtype": "hct_v3", "shape": [...], "data_offsets": [start, end]}}]
[data]; each tensor's bytes are a zstd frame (:389-391) around the fragment
container of its CompressiveSpectralEncoder fragments (:378-387): [u16 n] then
{u16 index, u16 flags, u64 XXH3-64 of the data, u32 len, data} per fragment.

TurboReader maps the file and decodes tensors on the GPU
(hh_turbo_tensor_decode) or hands their fragments to a progressive
StreamingTensorLoader.  TurboWriter is the producer; it stores each tensor's
zstd frame as raw blocks (valid RFC 8878 frames that every zstd decoder
reads; the reference compresses them at level 1, which changes nothing for a
reader)."""
import json
import mmap
import struct

from . import (BlockStatus, CHECKSUM_MISMATCH, CORRUPTED_DATA, F32, HaagentiError, OK, _addr, _lib, _sz, _u32,
               _torch_dtype, hct3_container, xxh3_64, xxh64, zstd_decompress)
import ctypes as C


def zstd_frame_raw(data):
    """A zstd frame of raw blocks with the content size and XXH64 checksum."""
    data = bytes(data)
    out = struct.pack("<IB", 0xFD2FB528, (3 << 6) | (1 << 5) | (1 << 2)) + struct.pack("<Q", len(data))
    blocks = [data[i:i + 131072] for i in range(0, len(data), 131072)] or [b""]
    for i, blk in enumerate(blocks):
        out += struct.pack("<I", (len(blk) << 3) | int(i == len(blocks) - 1))[:3] + blk
    return out + struct.pack("<I", xxh64(data) & 0xFFFFFFFF)


def parse_fragment_container(data):
    """[(index, flags, checksum, bytes)] of a fragment container (turbo.rs:378-387)."""
    data = bytes(data)
    if len(data) < 2:
        raise HaagentiError(CORRUPTED_DATA, "fragment container too short")
    n = struct.unpack_from("<H", data)[0]
    off, out = 2, []
    for _ in range(n):
        if len(data) - off < 16:
            raise HaagentiError(CORRUPTED_DATA, "truncated fragment header")
        idx, flags, chk, ln = struct.unpack_from("<HHQI", data, off)
        off += 16
        if ln > len(data) - off:
            raise HaagentiError(CORRUPTED_DATA, "fragment extends past the container")
        out.append((idx, flags, chk, data[off:off + ln]))
        off += ln
    return out


def dims(shape):
    """(width, height) as process_tensor_parallel derives them (turbo.rs:334-343)."""
    shape = [int(d) for d in shape]
    if len(shape) == 2:
        return shape[1], shape[0]
    if len(shape) == 1:
        return shape[0], 1
    total = 1
    for d in shape:
        total *= d
    w = shape[-1] if shape else 1
    return w, (total // w if w else 0)


class TurboWriter:
    """write_output (turbo.rs:421-463) for tensors given as encoder fragments."""

    def __init__(self):
        self._tensors = []

    def add_tensor(self, name, fragments, shape, dtype="hct_v3"):
        self._tensors.append((name, zstd_frame_raw(hct3_container(fragments)), list(shape), dtype))

    def to_bytes(self):
        meta, off = {}, 0
        for name, data, shape, dtype in self._tensors:
            meta[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(data)]}
            off += len(data)
        header = json.dumps(meta, separators=(",", ":")).encode()
        return struct.pack("<Q", len(header)) + header + b"".join(d for _, d, _, _ in self._tensors)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.to_bytes())


class TurboReader:
    """Reads a turbo output file through a memory map."""

    def __init__(self, path_or_bytes):
        self._map = None
        if isinstance(path_or_bytes, (bytes, bytearray, memoryview)):
            self._buf = memoryview(bytes(path_or_bytes))
            self._file = None
        else:
            self._file = open(path_or_bytes, "rb")
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
            self._buf = memoryview(self._map)
        if len(self._buf) < 8:
            raise HaagentiError(CORRUPTED_DATA, "turbo file too short")
        hl = struct.unpack_from("<Q", self._buf)[0]
        if 8 + hl > len(self._buf):
            raise HaagentiError(CORRUPTED_DATA, "turbo header past the end")
        self._meta = json.loads(bytes(self._buf[8:8 + hl]))
        self._data0 = 8 + hl

    def tensor_names(self):
        return list(self._meta)

    def info(self, name):
        m = self._meta[name]
        s, e = m["data_offsets"]
        return m["dtype"], list(m["shape"]), int(s), int(e)

    def tensor_bytes(self, name):
        _, _, s, e = self.info(name)
        if e < s or self._data0 + e > len(self._buf):
            raise HaagentiError(CORRUPTED_DATA, f"tensor {name} past the end of the file")
        return self._buf[self._data0 + s:self._data0 + e]

    def fragments(self, name, verify=True):
        """[(index, bytes)]: the tensor's zstd frame decoded on the host and its
        fragment container split (checksums verified when asked)."""
        frags = parse_fragment_container(zstd_decompress(bytes(self.tensor_bytes(name))))
        if verify:
            for idx, _, chk, data in frags:
                if xxh3_64(data) != chk:
                    raise HaagentiError(CHECKSUM_MISMATCH, f"fragment {idx} of {name}: checksum mismatch")
        return [(idx, data) for idx, _, _, data in frags]

    def decode_gpu(self, name, ctx, dtype=F32, d_out=None, verify=True, stream=None):
        """The whole tensor (every fragment) on the GPU: hh_turbo_tensor_decode."""
        import torch
        _, shape, _, _ = self.info(name)
        w, h = dims(shape)
        if d_out is None:
            d_out = torch.empty(max(w * h, 1), dtype=_torch_dtype(dtype), device="cuda")
        b = bytes(self.tensor_bytes(name))
        ww, hh, st = _u32(0), _u32(0), BlockStatus()
        rc = _lib.hh_turbo_tensor_decode(ctx.handle, b, len(b), 1 if verify else 0, int(dtype), _addr(d_out),
                                         d_out.numel(), C.byref(ww), C.byref(hh), C.byref(st), stream)
        if rc != OK:
            raise HaagentiError(rc, f"turbo tensor {name}", st)
        if (ww.value, hh.value) != (w, h):
            raise HaagentiError(CORRUPTED_DATA, f"tensor {name}: fragments are {ww.value}x{hh.value}, "
                                                f"shape gives {w}x{h}")
        return d_out[:w * h].view(*shape) if shape else d_out[:1]

    def streaming_loader(self, name, ctx=None):
        """A StreamingTensorLoader holding fragment 0 and the detail fragments queued."""
        from .streaming import StreamingTensorLoader
        _, shape, _, _ = self.info(name)
        w, h = dims(shape)
        frags = self.fragments(name)
        loader = StreamingTensorLoader(name, w, h, ctx=ctx)
        for f in frags:
            if f[0] == 0:
                loader.add_fragment(f)
        for f in reversed([f for f in frags if f[0] != 0]):
            loader.queue_fragment(f)      # load_next pops the most recently queued
        return loader

    def close(self):
        """Releases the map (views returned by tensor_bytes() must be gone)."""
        if self._buf is not None:
            self._buf.release()
            self._buf = None
        if self._map is not None:
            self._map.close()
            self._map = None
        if self._file:
            self._file.close()
            self._file = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
