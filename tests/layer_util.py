"""Producers for the decoder-layer tests: seeded N(0, 0.02) weights of a
layer's shapes stored as HCT-T tiles (one retention per tensor), cut into
LZ4 blocks of whole tiles (block size = the reference HctWriter's 16 KiB
default rounded down to whole tiles, crates/haagenti-hct/src/tensor.rs:74,536)
and compressed with the reference block compressor (host producer)."""
import numpy as np

L8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
       ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
L70B = [("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
        ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672)]


def encode_layer(H, shapes, ks, seed, block_bytes=16384):
    """Returns dict(blob, in_off, in_len, out_off, out_cap, tensors,
    scratch_bytes); every tensor keeps its tile bytes (`tiles`) and its
    offset in the scratch (`soff`)."""
    rng = np.random.default_rng(seed)
    comp = H.Lz4Compressor()
    parts, in_off, in_len, out_off, out_cap, tensors = [], [], [], [], [], []
    pos = spos = 0
    for (name, rows, cols), k in zip(shapes, ks):
        w = rng.standard_normal((rows, cols), dtype=np.float32)
        w *= np.float32(0.02)
        tiles = H.hctt_encode(w, k)
        del w
        tb = H.hctt_tile_bytes(k)
        blk = max(1, block_bytes // tb) * tb
        for s in range(0, tiles.size, blk):
            chunk = tiles[s:s + blk]
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
