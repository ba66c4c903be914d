"""Streaming decode runtime: PinnedBuffer, MemoryPool and
DecompressionPipeline (crates/haagenti-cuda/src/memory.rs:156-340,
crates/haagenti-cuda/src/pipeline.rs:35-320) over the C ABI
(hh_pinned_*, hh_pool_*, hh_pipeline_*).

The pipeline stages each unit (e.g. one decoder layer's LZ4 blocks) in a
page-locked buffer, copies it to the device on its copy stream and decodes
it on its compute stream; streams are ordered by events, so the copy of
unit l + 1 overlaps the decode of unit l."""
import ctypes as C

import numpy as np

from . import (BF16, OK, HaagentiError, HcttTensor, PipelineConfig, PipelineStats, PipelineTimes, PoolStats,
               BlockStatus, _addr, _check, _lib)

_vp = C.c_void_p


class PinnedBuffer:
    """PinnedBuffer (memory.rs:156-196): page-locked host memory."""

    def __init__(self, size):
        p = _vp()
        _check(_lib.hh_pinned_alloc(int(size), C.byref(p)), "hh_pinned_alloc")
        self._p, self._cap, self._size = p, int(size), int(size)

    def size(self):
        return self._size

    def as_array(self):
        """The whole buffer as a writable numpy uint8 array (no copy)."""
        if not self._cap:
            return np.zeros(0, np.uint8)
        return np.ctypeslib.as_array(C.cast(self._p, C.POINTER(C.c_uint8)), shape=(self._cap,))

    def as_slice(self):
        return self.as_array()[:self._size]

    def copy_from_host(self, src):
        """memory.rs:186-195: SizeMismatch (HH_ERR_INVALID_ARGUMENT) when src
        is larger than the buffer; the size becomes len(src)."""
        b = np.frombuffer(bytes(src), np.uint8) if not isinstance(src, np.ndarray) else src.view(np.uint8).ravel()
        if b.size > self._cap:
            raise HaagentiError(7, f"size mismatch: expected at most {self._cap}, got {b.size}")
        self.as_array()[:b.size] = b
        self._size = int(b.size)

    @property
    def address(self):
        return self._p.value

    def close(self):
        if getattr(self, "_p", None):
            _lib.hh_pinned_free(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuBuffer:
    """A piece of device memory from a MemoryPool (GpuBuffer, memory.rs:31-140)."""

    def __init__(self, ptr, size, pool):
        self.ptr, self._size, self.pool = int(ptr), int(size), pool

    def size(self):
        return self._size

    def data_ptr(self):
        return self.ptr


class MemoryPool:
    """MemoryPool (memory.rs:219-340): one device arena, first-fit pieces."""

    def __init__(self, ctx, total_size):
        p = _vp()
        _check(_lib.hh_pool_create(ctx.handle, int(total_size), C.byref(p)), "hh_pool_create")
        self._p, self.ctx = p, ctx

    @property
    def handle(self):
        return self._p

    def stats(self):
        s = PoolStats()
        _check(_lib.hh_pool_get_stats(self._p, C.byref(s)), "hh_pool_get_stats")
        return s

    def total_size(self):
        return self.stats().total_size

    def allocated(self):
        return self.stats().allocated

    def available(self):
        return self.stats().available

    def allocate(self, size, zero=True):
        """memory.rs:256-301 (zeroed, as alloc_zeros); OutOfMemory raises."""
        p = _vp()
        _check(_lib.hh_pool_allocate(self._p, int(size), 1 if zero else 0, C.byref(p)), "hh_pool_allocate")
        return GpuBuffer(p.value, size, self)

    def recycle(self, buf):
        _check(_lib.hh_pool_recycle(self._p, _vp(buf.ptr)), "hh_pool_recycle")

    def close(self):
        if getattr(self, "_p", None):
            _lib.hh_pool_destroy(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def default_config():
    c = PipelineConfig()
    _lib.hh_pipeline_default_config(C.byref(c))
    return c


def _u(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class DecompressionPipeline:
    """DecompressionPipeline (pipeline.rs:87-289) with event-ordered copy and
    compute streams.  `config` is a PipelineConfig (default_config() with
    the sizes filled in)."""

    def __init__(self, ctx, pool=None, config=None):
        cfg = config if config is not None else default_config()
        p = _vp()
        _check(_lib.hh_pipeline_create(ctx.handle, pool.handle if pool is not None else None, C.byref(cfg),
                                       C.byref(p)), "hh_pipeline_create")
        self._p, self.ctx, self.config, self._pool = p, ctx, cfg, pool
        # host arrays of submitted units, kept alive until the unit is waited
        # for: page-locked input is copied to the device from where it lies
        self._inflight = {}

    @property
    def streams(self):
        a, b = _vp(), _vp()
        _check(_lib.hh_pipeline_streams(self._p, C.byref(a), C.byref(b)))
        return a.value, b.value

    def next_staging(self):
        """The pinned staging buffer the next submit uses, as a numpy array
        (fill it in place to submit without a host copy)."""
        p, n = _vp(), C.c_size_t(0)
        _check(_lib.hh_pipeline_next_staging(self._p, C.byref(p), C.byref(n)), "hh_pipeline_next_staging")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(n.value,))

    def submit(self, data, in_off, in_len, out_off, out_cap, tensors=(), dtype=BF16, lz4_out=None, lz4_out_cap=0,
               after_event=None):
        """One unit: LZ4 blocks of `data` (a host uint8 array, possibly a
        view of next_staging()) -> the LZ4 output (`lz4_out`, or the tile
        scratch where the tensors' tiles are packed in order) -> the tensors,
        given as (tiles_len, rows, cols, k, d_out[, d_tile_status]).
        Returns the unit's ticket."""
        d = np.ascontiguousarray(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        assert d.dtype == np.uint8 and d.flags.c_contiguous
        io, il, oo, oc = _u(in_off, np.uint64), _u(in_len, np.uint32), _u(out_off, np.uint64), _u(out_cap, np.uint32)
        n = io.size
        arr = (HcttTensor * max(len(tensors), 1))()
        for i, t in enumerate(tensors):
            st = t[5] if len(t) > 5 else None
            arr[i] = HcttTensor(None, int(t[0]), int(t[1]), int(t[2]), int(t[3]), _addr(t[4]), _addr(st))
        tk = C.c_uint64(0)
        ev = after_event.cuda_event if hasattr(after_event, "cuda_event") else after_event
        _check(_lib.hh_pipeline_submit(self._p, d.ctypes.data if d.size else None, d.size, io.ctypes.data,
                                       il.ctypes.data, oo.ctypes.data, oc.ctypes.data, n, _addr(lz4_out),
                                       int(lz4_out_cap), arr, len(tensors), int(dtype), ev, C.byref(tk)),
               "hh_pipeline_submit")
        self._inflight[tk.value] = data
        return tk.value

    def wait(self, ticket):
        """Blocks until the unit is decoded; raises HaagentiError (with the
        failing block's record in .status and its index in .block) when a
        block failed."""
        st, fb = BlockStatus(), C.c_int64(-1)
        rc = _lib.hh_pipeline_wait(self._p, int(ticket), C.byref(st), C.byref(fb))
        for t in [t for t in self._inflight if t <= int(ticket)]:
            del self._inflight[t]   # units complete in order
        if rc != OK:
            e = HaagentiError(rc, f"unit {ticket} block {fb.value}", st)
            e.block = fb.value
            raise e

    def stream_wait(self, ticket, stream):
        _check(_lib.hh_pipeline_stream_wait(self._p, int(ticket), stream), "hh_pipeline_stream_wait")

    def times(self, ticket):
        t = PipelineTimes()
        _check(_lib.hh_pipeline_get_times(self._p, int(ticket), C.byref(t)), "hh_pipeline_get_times")
        return t

    def finish(self):
        """DecompressionPipeline::finish (pipeline.rs:262-269)."""
        st, fb, ft = BlockStatus(), C.c_int64(-1), C.c_uint64(0)
        rc = _lib.hh_pipeline_finish(self._p, C.byref(st), C.byref(fb), C.byref(ft))
        self._inflight.clear()
        if rc != OK:
            e = HaagentiError(rc, f"unit {ft.value} block {fb.value}", st)
            e.block, e.ticket = fb.value, ft.value
            raise e

    def stats(self):
        s = PipelineStats()
        _check(_lib.hh_pipeline_get_stats(self._p, C.byref(s)))
        return s

    def reset_stats(self):
        _lib.hh_pipeline_reset_stats(self._p)

    def close(self):
        if getattr(self, "_p", None):
            _lib.hh_pipeline_destroy(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
