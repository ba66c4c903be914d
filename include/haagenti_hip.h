/*
 * haagenti_hip.h -- C ABI of the MI355X (gfx950) HCT decode path.
 *
 * This is the boundary a `haagenti-hip` crate binds in place of
 * `haagenti-cuda`.  Every entry point names the reference interface it
 * replaces (file:line in the reference repository).  Signatures carry plain
 * pointers and sizes only: device pointers are prefixed d_, host pointers h_
 * (or unprefixed in host-only calls), streams are hipStream_t passed as
 * void* (NULL = HIP's null stream; hh_context_stream() gives the context's
 * own stream).
 *
 * Ownership: the caller allocates every input and output buffer.  A context
 * owns its device id, a stream, the IDCT basis table and a small scratch
 * pool; it is not thread-safe (one context per host thread), matching
 * GpuDctContext / GpuContext (crates/haagenti-cuda/src/lib.rs:99-108).
 * Device entry points are asynchronous on the given stream; results are
 * valid after that stream is synchronised.  A context's device scratch
 * (LZ4 scratch, whole-matrix transform buffers and tables) is shared by its
 * calls, so the asynchronous calls of one context must be ordered: the
 * same stream, or a synchronisation between calls made on different
 * streams.  Host-pointer entry points are
 * synchronous.  Every entry point makes the context's device current while
 * it runs and restores the calling thread's current device before it
 * returns.
 *
 * Errors: every entry returns an hh_status.  Kernels additionally write
 * per-block / per-tile status records (first error wins inside a block).
 */
#ifndef HAAGENTI_HIP_H
#define HAAGENTI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1-6 mirror haagenti_core::Error
 * (crates/haagenti-core/src/error.rs:10-60); 7-11 mirror CudaError
 * (crates/haagenti-cuda/src/error.rs:10-62). */
typedef enum hh_status {
    HH_OK = 0,
    HH_ERR_CORRUPTED_DATA = 1,    /* Error::CorruptedData */
    HH_ERR_BUFFER_TOO_SMALL = 2,  /* Error::BufferTooSmall {required, provided} */
    HH_ERR_UNEXPECTED_EOF = 3,    /* Error::UnexpectedEof {bytes_read} */
    HH_ERR_CHECKSUM_MISMATCH = 4, /* Error::ChecksumMismatch */
    HH_ERR_UNSUPPORTED = 5,       /* Error::Unsupported / CudaError::UnsupportedAlgorithm */
    HH_ERR_ALGORITHM = 6,         /* Error::Algorithm ("hct" container I/O) */
    HH_ERR_INVALID_ARGUMENT = 7,  /* CudaError::InvalidData / SizeMismatch */
    HH_ERR_OUT_OF_MEMORY = 8,     /* CudaError::OutOfMemory, Error::AllocationFailed */
    HH_ERR_DEVICE = 9,            /* CudaError::Driver / StreamSync */
    HH_ERR_KERNEL_LAUNCH = 10,    /* CudaError::KernelLaunch / KernelLoad */
    HH_ERR_DEVICE_NOT_FOUND = 11  /* CudaError::DeviceNotFound */
} hh_status;

/* Sub-kinds of HH_ERR_CORRUPTED_DATA (the reference's message strings). */
typedef enum hh_corrupt_kind {
    HH_CORRUPT_NONE = 0,
    HH_CORRUPT_ZERO_OFFSET = 1,    /* "invalid zero offset" (haagenti-lz4/src/block.rs:320-322) */
    HH_CORRUPT_OFFSET_BEYOND = 2,  /* "offset beyond output at offset N" (block.rs:323-325) */
    HH_CORRUPT_BITMAP_COUNT = 3,   /* "bitmap has N set bits, expected K" (compressive.rs:630-636) */
    HH_CORRUPT_HEADER = 4,         /* invalid magic/version/algorithm/dtype (tensor.rs:311-331) */
    HH_CORRUPT_SIZE = 5,           /* sizes inconsistent with the header/shape */
    HH_CORRUPT_HEADER_CHECKSUM = 6,  /* "header checksum mismatch" (haagenti-hct/src/tensor.rs:857-865) */
    HH_CORRUPT_BLOCK_CHECKSUM = 7,   /* "block N checksum mismatch" (tensor.rs:965-974) */
    HH_CORRUPT_QUANT_SCHEME = 8      /* "unknown quantization scheme" (tensor.rs:158-173) */
} hh_corrupt_kind;

/* Output element types; values match haagenti_hct::DType (tensor.rs:99-105). */
typedef enum hh_dtype { HH_F32 = 0, HH_F16 = 1, HH_BF16 = 2 } hh_dtype;

/* Per-block status written by device kernels (32 bytes). */
typedef struct hh_block_status {
    int32_t code;      /* hh_status */
    int32_t detail;    /* hh_corrupt_kind when code == HH_ERR_CORRUPTED_DATA */
    uint64_t position; /* UnexpectedEof: bytes_read; OffsetBeyond: output position */
    uint64_t required; /* BufferTooSmall: required output bytes */
    uint64_t written;  /* bytes produced (valid when code == HH_OK) */
} hh_block_status;

typedef struct hh_context hh_context;

/* ---------------------------------------------------------------- misc */

/* Error::category() strings (crates/haagenti-core/src/error.rs:120-134). */
const char *hh_status_category(int32_t code);
/* Error::is_recoverable() (error.rs:112-117): UnexpectedEof, BufferTooSmall. */
int32_t hh_status_is_recoverable(int32_t code);
const char *hh_version(void);
/* Number of visible devices (haagenti_cuda::is_available, lib.rs:233). */
int32_t hh_device_count(void);

/* GpuContext::new / GpuDecompressor::new(device_id)
 * (crates/haagenti-cuda/src/lib.rs:112-142, decompress.rs:117-127). */
int32_t hh_context_create(int32_t device, hh_context **out);
void hh_context_destroy(hh_context *ctx);
/* The context's stream (hipStream_t) as void*. */
void *hh_context_stream(hh_context *ctx);
int32_t hh_context_synchronize(hh_context *ctx);

/* Context settings for diagnostics and tests; no counterpart in the
 * reference (whose GPU contexts have no tunables).  HH_OPT_LZ4_DECODER
 * selects the LZ4 block decoder of every batched LZ4 launch made through the
 * context (hh_lz4_decoder), and the block decoder of the fused layer entries
 * (HH_LZ4_SEQ or one of the ring decoders, which decode there into LDS).
 * The default, HH_LZ4_AUTO, takes the one-sequence ring decoder (4 KiB
 * ring) for hh_lz4_decompress_batch, and for the layer entries (two-launch,
 * fused, no-alloc, hh_pipeline_submit) the sequence-batched decoder when a
 * tensor of the call has k < 1024 (retention below 25 %: its tiles compress
 * into blocks of many short LZ4 sequences) and the ring decoder otherwise
 * (denser tiles leave a few long runs per block).  HH_OPT_FUSED_POLL_LIMIT bounds every wait of
 * the fused layer decode to that many polls (1 .. 2^24; 0 restores 2^24),
 * so a test can drive the path taken when a wait runs out.
 * HH_OPT_DCT_ROUTE picks the whole-matrix transform of hh_idct_2d,
 * hh_dct_2d and the HCT3 decode entries (hh_dct_route): HH_DCT_AUTO (the
 * default) takes the FFT route when both sides allow it and the larger is
 * at least 1024, the dense MFMA products otherwise.
 * HH_OPT_PIPELINE_ROUTE picks how hh_pipeline_submit decodes a unit's
 * tensors (hh_pipeline_route): HH_PIPE_AUTO (the default) decodes each
 * tensor with k >= 1024 whose blocks hold whole tiles in the fused launch
 * (hh_hctt_decode_lz4_fused) and the others through the LZ4 launch and the
 * tile launch; HH_PIPE_TWO_LAUNCH takes the two launches for every tensor;
 * HH_PIPE_FUSED the fused launch for every tensor whose blocks allow it.
 * Returns HH_ERR_INVALID_ARGUMENT for an unknown option or value. */
typedef enum hh_option {
    HH_OPT_LZ4_DECODER = 1,
    HH_OPT_FUSED_POLL_LIMIT = 2,
    HH_OPT_DCT_ROUTE = 3,
    HH_OPT_PIPELINE_ROUTE = 4
} hh_option;
typedef enum hh_pipeline_route { HH_PIPE_AUTO = 0, HH_PIPE_TWO_LAUNCH = 1, HH_PIPE_FUSED = 2 } hh_pipeline_route;
typedef enum hh_dct_route {
    HH_DCT_AUTO = 0,
    HH_DCT_DENSE = 1, /* split-f16 MFMA products against cached bases, O(n^3) */
    HH_DCT_FFT = 2    /* row transforms through an FFT, O(n^2 log n), where the sides allow it */
} hh_dct_route;
typedef enum hh_lz4_decoder {
    HH_LZ4_AUTO = 0,   /* per entry point, as above */
    HH_LZ4_SEQ = 1,    /* sequences parsed in batches, copies lane-parallel; 4 KiB ring */
    HH_LZ4_SEQ8 = 2,   /* the same with an 8 KiB ring */
    HH_LZ4_RING4 = 3,  /* one sequence at a time through a 4 KiB LDS ring */
    HH_LZ4_RING8 = 4,
    HH_LZ4_RING16 = 5,
    HH_LZ4_RING32 = 6,
    HH_LZ4_WINDOW = 7  /* one sequence at a time, global -> global */
} hh_lz4_decoder;
int32_t hh_context_set_option(hh_context *ctx, int32_t option, int64_t value);

/* Streaming device-to-device copy of `bytes` bytes (non-overlapping ranges):
 * no counterpart in the reference; it is the bandwidth calibration of this
 * library's measurements (the rate a kernel that reads and writes every byte
 * once can reach on the device, and the scale of the FETCH_SIZE /
 * WRITE_SIZE counters).  Asynchronous on the stream. */
int32_t hh_hbm_copy(hh_context *ctx, void *d_dst, const void *d_src, uint64_t bytes, void *stream);

/* ---------------------------------------------------------------- LZ4 */

/* Batched raw-LZ4 block decode, one wavefront per block.  Block i reads
 * d_in[d_in_off[i] .. +d_in_len[i]) and writes at most d_out_cap[i] bytes
 * at d_out + d_out_off[i]; d_out_cap[i] is both output.len() and
 * output_size of decompress_block (haagenti-lz4/src/block.rs:261-366).
 * in_total bounds every input read (size of the d_in allocation).
 * d_status[i] receives the block's result; a stream that ends early is
 * success with written < cap, as in the reference.  A block that fails
 * leaves its whole output range [d_out_off[i], +d_out_cap[i]) zeroed (the
 * reference returns an error and no output).
 * Replaces NativeKernels::decompress_lz4_native
 * (crates/haagenti-cuda/src/native_kernels.rs:623-657) and
 * GpuContext::decompress_lz4 (lib.rs:173-197). */
int32_t hh_lz4_decompress_batch(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                const uint64_t *d_in_off, const uint32_t *d_in_len,
                                uint8_t *d_out, const uint64_t *d_out_off,
                                const uint32_t *d_out_cap, uint32_t nblocks,
                                hh_block_status *d_status, void *stream);

/* Host-pointer, single block: Decompressor::decompress_to
 * (haagenti-core/src/traits.rs:80; haagenti-lz4/src/decompress.rs:59-61),
 * decoded on the GPU.  Synchronous.  *status receives the full record. */
int32_t hh_lz4_decompress_to(hh_context *ctx, const uint8_t *in, size_t in_len,
                             uint8_t *out, size_t out_cap, size_t *written,
                             hh_block_status *status);

/* Compressor::compress_to with the LZ4 block compressor
 * (haagenti-lz4/src/block.rs:73-147; compress.rs:81-99), on the host.
 * Byte-identical output.  *written receives the compressed size;
 * HH_ERR_BUFFER_TOO_SMALL with *written = required when out_cap is short. */
int32_t hh_lz4_compress_block(const uint8_t *in, size_t in_len, uint8_t *out,
                              size_t out_cap, size_t *written);
/* block.rs:370-373 */
size_t hh_lz4_max_compressed_size(size_t input_len);

/* ---------------------------------------------------------------- INT4 */

/* testing::dequantize_int4 (crates/haagenti/src/testing/quantization.rs:82-131)
 * on the GPU: d_q = [ceil(n/32) f16 scales][ceil(n/2) nibble bytes],
 * q_len bytes.  Writes *produced = min(n, 2*(q_len - scale bytes))
 * elements (0 when q_len is shorter than the scales), as the reference's
 * early stop does.  HH_F32 output is bit-identical to the reference;
 * HH_BF16 / HH_F16 are the round-to-nearest-even of that f32.
 * Replaces NativeKernels::dequantize_int4_fp16 (native_kernels.rs:694-729),
 * whose signed-nibble fp16 arithmetic disagrees with the CPU format. */
int32_t hh_dequant_int4(hh_context *ctx, const uint8_t *d_q, size_t q_len, size_t n,
                        int32_t out_dtype, void *d_out, size_t *produced, void *stream);

/* testing::quantize_int4 (quantization.rs:30-70) on the host (producer
 * side).  out must hold hh_int4_compressed_size(n) bytes. */
size_t hh_quantize_int4(const float *w, size_t n, uint8_t *out);
size_t hh_int4_compressed_size(size_t n); /* quantization.rs:202-210 */

/* ---------------------------------------------------------------- HCT-T tiles */

/* Bytes of one 64x64 HCT-T tile with k retained coefficients:
 * 512-byte bitmap + ceil(k/32) f16 scales + ceil(k/2) nibble bytes. */
size_t hh_hctt_tile_bytes(uint32_t k);
/* Retained count for a retention ratio: max(1, (4096 as f32 * clamp(rho,
 * 0.05, 1)) as usize) (crates/haagenti/src/compressive.rs:97,152). */
uint32_t hh_hctt_retain_count(float rho);

/* Decode a rows x cols tensor stored as row-major 64x64 HCT-T tiles:
 * per tile dequantize_int4 -> bitmap scatter (compressive.rs:620-627,
 * 741-745) -> 2-D inverse DCT (haagenti-core/src/dct.rs:311-337), on MFMA.
 * d_tile_status (optional, one int32 per tile) receives HH_OK or
 * HH_ERR_CORRUPTED_DATA (bitmap popcount != k; that tile is written as
 * zeros).  Output row-major rows x cols of out_dtype; rows and cols are
 * multiples of 64, cols at most 2^24 (else HH_ERR_INVALID_ARGUMENT).
 * Replaces GpuDctContext::idct_2d_gpu (crates/haagenti-cuda/src/dct_gpu.rs:1163)
 * and GpuDecompressor::decompress_to_gpu (decompress.rs:183-203). */
int32_t hh_hctt_decode(hh_context *ctx, const uint8_t *d_tiles, size_t tiles_len,
                       uint32_t rows, uint32_t cols, uint32_t k, int32_t out_dtype,
                       void *d_out, int32_t *d_tile_status, void *stream);

/* One tensor of a batched decode (device pointers; the array itself is
 * host memory and is consumed before the call returns). */
typedef struct hh_hctt_tensor {
    const uint8_t *d_tiles;
    size_t tiles_len;
    uint32_t rows, cols, k;
    void *d_out;
    int32_t *d_tile_status; /* optional */
} hh_hctt_tensor;

/* Several tensors (e.g. all weights of one decoder layer, each with its own
 * retention k) in as few launches as possible, same output dtype.  Same
 * per-tensor semantics as hh_hctt_decode; this is the batched form of
 * GpuDecompressor::decompress_batch_to_gpu (decompress.rs:282-293). */
int32_t hh_hctt_decode_batch(hh_context *ctx, const hh_hctt_tensor *tensors, uint32_t n,
                             int32_t out_dtype, void *stream);

/* LZ4-compressed HCT-T tiles of several tensors in one call: every block of
 * d_in is decoded into d_scratch (hh_lz4_decompress_batch semantics, one
 * status record per block in d_status), then the tensors, whose d_tiles point
 * into d_scratch, are decoded (hh_hctt_decode_batch semantics); both launches
 * are queued on `stream` with no host synchronization.  This is what
 * HctReader::decompress_all (haagenti-hct/src/tensor.rs:417-515) followed by
 * GpuDecompressor::decompress_batch_to_gpu (haagenti-cuda/src/decompress.rs:
 * 282-293) does for one layer's tensors.  A block that fails leaves its
 * range of d_scratch zeroed, so every tile it covers fails the bitmap count
 * (tile status HH_ERR_CORRUPTED_DATA, output zeros) whatever the scratch held
 * before; d_status names the block once the stream completes.  A block that
 * decodes short (HH_OK, fewer bytes than its capacity) zeroes the rest of
 * its range, so the tiles there fail the same way (as in
 * hh_hctt_decode_lz4_fused and the no-alloc entry). */
int32_t hh_hctt_decode_lz4_batch(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                 const uint64_t *d_in_off, const uint32_t *d_in_len,
                                 uint8_t *d_scratch, const uint64_t *d_out_off,
                                 const uint32_t *d_out_cap, uint32_t nblocks,
                                 hh_block_status *d_status, const hh_hctt_tensor *tensors,
                                 uint32_t ntensors, int32_t out_dtype, void *stream);

/* hh_hctt_decode_lz4_batch in one launch with the tile bytes kept on chip:
 * HctReader::decompress_all (haagenti-hct/src/tensor.rs:417-515) and
 * GpuDecompressor::decompress_batch_to_gpu (haagenti-cuda/src/decompress.rs:
 * 282-293) fused, no d_scratch.  Each LZ4 block holds whole tiles of one
 * tensor: tensor i's blocks are the next ceil(ntiles_i / tiles_per_block)
 * entries of d_in_off / d_in_len (tensor 0's first), each decompressing to
 * tiles_per_block tiles (a tensor's last block to the rest), at most
 * HH_FUSED_BLOCK_BYTES of tile bytes per block (HH_ERR_UNSUPPORTED
 * otherwise); nblocks must be their total.  tensors[i].d_tiles / tiles_len
 * are not used.  d_status receives one record per block as
 * hh_lz4_decompress_batch writes it (the expected size is the block's tile
 * bytes); the tile bytes a block does not produce (all of a failed block's)
 * read as zeros, so those tiles report HH_ERR_CORRUPTED_DATA with zero
 * output.  Asynchronous on the stream.  One persistent workgroup per CU
 * takes every G-th block (G workgroups) and its tiles: each of its waves in
 * turn decodes the next of those blocks into an LDS block buffer (when one
 * is free) or the next of their tiles from the buffers.  Every wait between
 * the waves is bounded (HH_OPT_FUSED_POLL_LIMIT polls); when one runs out,
 * every block record and every tile status of that workgroup's blocks
 * report HH_ERR_DEVICE and those tiles' outputs are unspecified (the
 * kernel still ends; the next call decodes normally).  One launch takes up
 * to 32 tensors (more go to further launches of up to 32, in order); a
 * launch has a fixed cost (its workgroups' start, the first blocks' decode,
 * the last tiles' drain) of about 10 us on an MI355X, so several layers'
 * tensors passed in one call, their blocks in one buffer, decode faster
 * than one call per layer. */
#define HH_FUSED_BLOCK_BYTES 16352u
int32_t hh_hctt_decode_lz4_fused(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                 const uint64_t *d_in_off, const uint32_t *d_in_len, uint32_t nblocks,
                                 hh_block_status *d_status, const hh_hctt_tensor *tensors, uint32_t ntensors,
                                 uint32_t tiles_per_block, int32_t out_dtype, void *stream);

/* hh_hctt_decode_lz4_fused with tiles_per_block[i] tiles per LZ4 block of
 * tensor i: each tensor written by its own HctWriter whose block size
 * (HctWriter::with_block_size, haagenti-hct/src/tensor.rs:544-547; chunks of
 * it compressed one by one, :556-561) is a whole number of that tensor's
 * tiles, e.g. floor(16384 / tile bytes) tiles in a layer of mixed k. */
int32_t hh_hctt_decode_lz4_fused_tpb(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                     const uint64_t *d_in_off, const uint32_t *d_in_len, uint32_t nblocks,
                                     hh_block_status *d_status, const hh_hctt_tensor *tensors, uint32_t ntensors,
                                     const uint32_t *tiles_per_block, int32_t out_dtype, void *stream);

/* Size of the tile-byte array hh_hctt_decode_lz4_batch_noalloc uses: 64 MiB
 * (a Llama-3-8B layer's tiles at 30 % retention take 64,110,592 bytes). */
#define HH_NOALLOC_SCRATCH_BYTES (64ull << 20)

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  hh_hctt_decode_lz4_batch with the LZ4 output held in a
 * device array the library owns (HH_NOALLOC_SCRATCH_BYTES per GPU, held
 * until the process ends) instead of a caller's d_scratch; it allocates
 * nothing.  Every tensors[i].d_tiles must be NULL: the tensors' tiles are
 * packed in order from the array's start (tensor i's at byte offset
 * sum_{j<i} tiles_len_j), and d_out_off are offsets into the array.  More
 * than HH_NOALLOC_SCRATCH_BYTES of tiles_len in total is
 * HH_ERR_BUFFER_TOO_SMALL (nothing is launched); a block whose output range
 * leaves the packed tiles gets HH_ERR_INVALID_ARGUMENT in d_status and
 * writes nothing.  All calls on one GPU share its array and it keeps the
 * last call's bytes: calls that overlap on one GPU race, and tile bytes no
 * block covers hold an earlier call's data. */
int32_t hh_hctt_decode_lz4_batch_noalloc(hh_context *ctx, const uint8_t *d_in, size_t in_total,
                                         const uint64_t *d_in_off, const uint32_t *d_in_len,
                                         const uint64_t *d_out_off, const uint32_t *d_out_cap,
                                         uint32_t nblocks, hh_block_status *d_status,
                                         const hh_hctt_tensor *tensors, uint32_t ntensors,
                                         int32_t out_dtype, void *stream);

/* Producer side on the host (threads = 0: all cores): per tile
 * dct_2d (dct.rs:282-308) -> top-k by |c| (compressive.rs:144-172) ->
 * quantize_int4 of the kept coefficients in ascending index order. */
int32_t hh_hctt_encode(const float *w, uint32_t rows, uint32_t cols, uint32_t k,
                       uint8_t *out, int32_t threads);

/* ---------------------------------------------------------------- streaming */

/* PinnedBuffer::new (crates/haagenti-cuda/src/memory.rs:156-196), as page-
 * locked host memory (hipHostMalloc; the reference's is a Vec placeholder,
 * memory.rs:161-168).  bytes = 0 gives *out = NULL. */
int32_t hh_pinned_alloc(size_t bytes, void **out);
int32_t hh_pinned_free(void *ptr);

/* MemoryPool (memory.rs:200-340): one device arena of total_size bytes
 * (allocated once at creation), handed out in 256-byte-aligned pieces,
 * first fit, freed pieces coalesced.  Not thread-safe across pools; one
 * pool may be used from several threads. */
typedef struct hh_pool hh_pool;
typedef struct hh_pool_stats { /* PoolStats (memory.rs:341-347) */
    uint64_t total_size;
    uint64_t allocated;
    uint64_t available;          /* MemoryPool::available (memory.rs:251-254) */
    uint64_t free_buffers;       /* free extents */
    uint64_t free_buffer_bytes;
    uint64_t largest_free;       /* the largest piece allocate() can return */
} hh_pool_stats;
int32_t hh_pool_create(hh_context *ctx, size_t total_size, hh_pool **out);
void hh_pool_destroy(hh_pool *pool);
/* MemoryPool::allocate (memory.rs:256-301): HH_ERR_OUT_OF_MEMORY when no
 * free extent holds size bytes; zero != 0 clears the piece (the reference
 * hands out zeroed buffers) with a synchronous memset. */
int32_t hh_pool_allocate(hh_pool *pool, size_t size, int32_t zero, void **d_out);
/* MemoryPool::recycle (memory.rs:312-317): the piece returns to the pool. */
int32_t hh_pool_recycle(hh_pool *pool, void *d_ptr);
int32_t hh_pool_get_stats(hh_pool *pool, hh_pool_stats *out);

/* DecompressionPipeline (crates/haagenti-cuda/src/pipeline.rs:87-289):
 * units of compressed LZ4 blocks (a decoder layer's tensors) staged in
 * page-locked host buffers, copied to the device on a copy stream and
 * decoded on a compute stream, ordered by events only, so the copy of unit
 * l + 1 runs under the decode of unit l.  The reference synchronises the
 * device between stages (pipeline.rs:212-232). */
typedef struct hh_pipeline hh_pipeline;
typedef struct hh_pipeline_config { /* PipelineConfig (pipeline.rs:35-60) */
    uint32_t num_staging_buffers; /* 2 = double buffering (1..16) */
    uint32_t max_blocks;          /* LZ4 blocks per unit */
    uint64_t staging_buffer_size; /* bytes of one unit: data + 24 bytes per block of tables */
    uint64_t tile_scratch_size;   /* device bytes for a unit's LZ4 output (tile bytes) */
    uint32_t use_pinned_memory;   /* 1: hipHostMalloc staging */
    uint32_t copy_threads;        /* host threads that copy a unit into staging */
} hh_pipeline_config;
typedef struct hh_pipeline_stats { /* PipelineStats (pipeline.rs:121-128) */
    uint64_t blocks_processed;
    uint64_t bytes_read;          /* compressed bytes copied to the device */
    uint64_t bytes_decompressed;  /* LZ4 output bytes */
    uint64_t transfer_time_ns;    /* host -> device copies (copy-stream events) */
    uint64_t decompress_time_ns;  /* LZ4 + tile decode (compute-stream events) */
    uint64_t units;               /* units completed */
    uint64_t bytes_output;        /* decoded tensor bytes */
} hh_pipeline_stats;
/* Event times of one unit, in milliseconds since the pipeline's creation. */
typedef struct hh_pipeline_times {
    double h2d_start_ms, h2d_end_ms, decode_start_ms, decode_end_ms;
} hh_pipeline_times;

/* PipelineConfig::default: 2 staging buffers of 4 MiB, 65536 blocks, no
 * tile scratch, pinned memory, 8 copy threads. */
void hh_pipeline_default_config(hh_pipeline_config *cfg);
/* DecompressionPipeline::new (pipeline.rs:134-170): the staging buffers,
 * their device copies, per-slot status records and events, and the tile
 * scratch; device memory comes from `pool` when given, else hipMalloc. */
int32_t hh_pipeline_create(hh_context *ctx, hh_pool *pool, const hh_pipeline_config *cfg, hh_pipeline **out);
void hh_pipeline_destroy(hh_pipeline *p);
/* The pipeline's copy and compute streams (hipStream_t as void*). */
int32_t hh_pipeline_streams(hh_pipeline *p, void **copy_stream, void **compute_stream);
/* The staging buffer the next hh_pipeline_submit uses (after the unit that
 * last used it has completed), for callers that read their data straight
 * into it (PinnedBuffer::as_mut_slice); submitting from there copies
 * nothing on the host. */
int32_t hh_pipeline_next_staging(hh_pipeline *p, uint8_t **h_ptr, size_t *cap);
/* DecompressionPipeline::submit_block + process (pipeline.rs:178-259) for
 * one unit: h_data[0, len) holds nblocks LZ4 blocks (block i at h_in_off[i],
 * h_in_len[i] bytes), decoded to d_lz4_out (lz4_out_cap bytes; NULL: the
 * pipeline's tile scratch) at h_out_off[i], at most h_out_cap[i] bytes
 * (hh_lz4_decompress_batch semantics).  Then the tensors (their d_tiles
 * NULL: their tiles are packed in order in the LZ4 output) are decoded as
 * hh_hctt_decode_batch does.  after_event (a hipEvent_t, or NULL) delays
 * the decode until it completes (e.g. the consumer of the tensors' output
 * slot is done with it).  The host blocks only while the staging slot's
 * previous unit completes.  *ticket names the unit.
 * Lifetime of h_data: pageable memory is copied into the slot's staging
 * buffer before the call returns, so the caller may reuse it at once.
 * Page-locked memory (hh_pinned_alloc, hipHostMalloc, a pinned torch
 * tensor) is copied to the device from where it lies, with no host copy:
 * it must stay allocated and unchanged until the unit has been waited for
 * (hh_pipeline_wait / hh_pipeline_finish) or its stream event passed
 * (hh_pipeline_stream_wait).  Every tensor is checked (shape, k, tile
 * bytes, output alignment) before anything is enqueued; an invalid one
 * fails the call with nothing enqueued.
 * Route: with d_lz4_out NULL, a tensor whose blocks cut its packed tile
 * bytes into runs of tiles_per_block whole tiles (ascending, the last run
 * the rest, at most HH_FUSED_BLOCK_BYTES each) may be decoded by the fused
 * launch, its tile bytes then never written to the scratch
 * (HH_OPT_PIPELINE_ROUTE; by default the tensors with k >= 1024).  Outputs,
 * tile statuses and block records are the same either way. */
int32_t hh_pipeline_submit(hh_pipeline *p, const uint8_t *h_data, size_t len, const uint64_t *h_in_off,
                           const uint32_t *h_in_len, const uint64_t *h_out_off, const uint32_t *h_out_cap,
                           uint32_t nblocks, uint8_t *d_lz4_out, uint64_t lz4_out_cap,
                           const hh_hctt_tensor *tensors, uint32_t ntensors, int32_t out_dtype,
                           void *after_event, uint64_t *ticket);
/* Blocks until the unit is decoded; returns its first failing block's code
 * (HH_OK when every block decoded), with that block's record and index.
 * Each ticket can be waited for once. */
int32_t hh_pipeline_wait(hh_pipeline *p, uint64_t ticket, hh_block_status *status, int64_t *failed_block);
/* Makes `stream` wait (on the device) for the unit's decode. */
int32_t hh_pipeline_stream_wait(hh_pipeline *p, uint64_t ticket, void *stream);
/* The unit's copy and decode intervals (waits for it). */
int32_t hh_pipeline_get_times(hh_pipeline *p, uint64_t ticket, hh_pipeline_times *out);
/* DecompressionPipeline::finish (pipeline.rs:262-269): waits for every
 * unit; returns the first failure among the units not waited for. */
int32_t hh_pipeline_finish(hh_pipeline *p, hh_block_status *status, int64_t *failed_block, uint64_t *failed_ticket);
/* DecompressionPipeline::stats / reset_stats (pipeline.rs:281-289). */
int32_t hh_pipeline_get_stats(hh_pipeline *p, hh_pipeline_stats *out);
void hh_pipeline_reset_stats(hh_pipeline *p);

/* ---------------------------------------------------------------- HCT container */

/* Header and block-index geometry of an HCT v1 file (64-byte header,
 * tensor.rs:275-375; 8-byte block index entries, :379-405). */
typedef struct hh_hct_info {
    uint32_t version;
    uint8_t algorithm;      /* 0 LZ4, 1 Zstd (tensor.rs CompressionAlgorithm) */
    uint8_t dtype;          /* haagenti_hct::DType, 0..4 */
    uint16_t flags;
    uint64_t original_size;
    uint64_t compressed_size;
    uint32_t block_size;
    uint32_t num_blocks;
    uint32_t rank;
    uint32_t index_entry_size; /* 8, or 16 for v2 files with block checksums */
    uint64_t shape[4];
    uint64_t data_offset;   /* header + quantization metadata + index */
} hh_hct_info;

/* QuantizationMetadata of HCT v2 (tensor.rs:180-226), 8 bytes after the
 * header when flags has 0x0004. */
typedef struct hh_hct_quant {
    uint8_t present;
    uint8_t scheme;         /* QuantizationScheme 0..4 (tensor.rs:144-156) */
    uint8_t has_per_group_scales;
    int8_t zero_point;
    uint16_t scale_bits;    /* f16 bits */
    uint16_t pad;
    uint32_t group_size;    /* 24 bits on disk */
} hh_hct_quant;

/* HctHeader::from_bytes (crates/haagenti-hct/src/tensor.rs:302-375) and the
 * index read of HctReader::new (:417-445) on host bytes.  Errors as the
 * reference reports them: a file shorter than the header or its index is
 * HH_ERR_ALGORITHM (read_exact failures, :420-431); bad magic, version > 2,
 * unknown algorithm or dtype, or a rank above 3 are HH_ERR_CORRUPTED_DATA
 * with detail HH_CORRUPT_HEADER (status, when given, receives the record). */
int32_t hh_hct_read_header(const uint8_t *file, size_t file_len, hh_hct_info *info,
                           hh_block_status *status);

/* HctReader::new + decompress_all with the LZ4 decompressor
 * (tensor.rs:417-515): every block of the file decoded in one batched GPU
 * launch.  h_file is the file on the host (at least its header and index;
 * file_len is the full length), d_file the same file in device memory.  The
 * output is the concatenation of the blocks as the reference builds it (a
 * block that decodes short shifts the ones after it) in d_out (out_cap
 * bytes); *written receives its length.  On failure the error is the one
 * the reference's block-by-block loop meets first: an index entry past the
 * end of the file (HH_ERR_ALGORITHM, :477-480), an inconsistent last-block
 * size (HH_ERR_CORRUPTED_DATA / HH_CORRUPT_SIZE, :494-500), output beyond
 * out_cap (HH_ERR_BUFFER_TOO_SMALL), or the block's LZ4 error; *failed_block
 * (optional) receives its index, or -1.  Synchronous on the given stream. */
int32_t hh_hct_decompress_all(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                              size_t file_len, uint8_t *d_out, size_t out_cap, size_t *written,
                              hh_block_status *status, int64_t *failed_block, void *stream);

/* ---- HCT v2: XXH3-64 checksums (tensor.rs:45-271, 676-1021) ------------ */

/* xxhash_rust::xxh3::xxh3_64 (xxhash-rust 0.8.15, seed 0) as called at
 * tensor.rs:729,794,858,967, on host memory. */
uint64_t hh_xxh3_64(const uint8_t *data, size_t len);

/* The same hash of n device buffers data[off[i], off[i] + len[i]) in one
 * launch (one wavefront per buffer), into d_out[i].  A range outside
 * [0, data_len) yields 0.  Asynchronous on the stream.  Replaces the
 * per-block xxh3_64 of HctReaderV2::read_block_validated (:965-974). */
int32_t hh_xxh3_64_batch(hh_context *ctx, const uint8_t *d_data, size_t data_len,
                         const uint64_t *d_off, const uint32_t *d_len, uint32_t n, uint64_t *d_out,
                         void *stream);

/* HctReaderV2::new (tensor.rs:841-920) on host bytes: the v1 header checks,
 * then the header checksum (version >= 2 and flags & 0x0001: XXH3 of bytes
 * 0..56 must equal bytes 56..64, else HH_ERR_CORRUPTED_DATA /
 * HH_CORRUPT_HEADER_CHECKSUM), the quantization metadata (flags & 0x0004;
 * short file HH_ERR_ALGORITHM, unknown scheme HH_CORRUPT_QUANT_SCHEME), and
 * the index entry size (16 when version >= 2 and flags & 0x0002, else 8).
 * quant may be NULL. */
int32_t hh_hct_read_header_v2(const uint8_t *file, size_t file_len, hh_hct_info *info,
                              hh_hct_quant *quant, hh_block_status *status);

/* HctReaderV2::new + decompress_all_validated (tensor.rs:980-1012): as
 * hh_hct_decompress_all, with every block's XXH3 (when its index entry
 * holds a non-zero checksum) computed on the GPU in one launch and checked
 * in the reference's per-block order: index range (HH_ERR_ALGORITHM), then
 * checksum (HH_ERR_CORRUPTED_DATA / HH_CORRUPT_BLOCK_CHECKSUM), then size,
 * output capacity and the block's LZ4 result.  Synchronous on the stream. */
int32_t hh_hct_decompress_all_validated(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                                        size_t file_len, uint8_t *d_out, size_t out_cap,
                                        size_t *written, hh_block_status *status,
                                        int64_t *failed_block, void *stream);

/* HctReaderV2::new + validate_checksums (tensor.rs:1014-1020): the header
 * checks and every block's range and checksum, without decoding. */
int32_t hh_hct_validate_checksums(hh_context *ctx, const uint8_t *h_file, const uint8_t *d_file,
                                  size_t file_len, hh_block_status *status, int64_t *failed_block,
                                  void *stream);

/* ------------------------------------------- HCT3 whole-tensor spectral */

/* HCT V3 fragment container (the layout GpuDecompressor and the reference C
 * decoder read): [u16 n] then n x {u16 index, u16 flags, u64 checksum,
 * u32 len, len bytes}; a fragment's bytes are [u32 count][ceil(total/8)
 * bitmap][f16 values]. */

/* GpuDecompressor::parse_hct_fragments + reconstruct_coefficients
 * (crates/haagenti-cuda/src/decompress.rs:322-427) on the GPU: the dense
 * DCT coefficient matrix (total f32) of a container held in host memory.
 * A fragment that ends past the data is HH_ERR_INVALID_ARGUMENT
 * (CudaError::InvalidData); fragments shorter than 4 + bitmap bytes are
 * skipped; each fragment's values fill its set bits in ascending order
 * while they last, later fragments overwriting earlier ones.  zstd-framed
 * input (magic 28 B5 2F FD, the turbo wrapper) is first decoded on the host
 * (hh_zstd_decompress); when that fails the bytes are parsed as a raw
 * container, as try_zstd_decompress does (decompress.rs:296-319).
 * Synchronous. */
int32_t hh_hct3_coefficients(hh_context *ctx, const uint8_t *data, size_t len, uint64_t total,
                             float *d_coeffs, void *stream);

/* GpuDecompressor::decompress / decompress_to_gpu (decompress.rs:153-192):
 * the coefficients as above, then the orthonormal inverse DCT of the whole
 * height x width matrix (width = last dimension, height = product of the
 * others, decompress.rs:430-442; idct_2d, haagenti-core/src/dct.rs:311-337)
 * into d_out (product(shape) elements of out_dtype).  Synchronous. */
int32_t hh_hct3_decompress(hh_context *ctx, const uint8_t *data, size_t len, const uint64_t *shape,
                           uint32_t rank, int32_t out_dtype, void *d_out, void *stream);

/* hh_hct3_decompress with the container also resident in device memory
 * (d_data, a copy of h_data; h_data is parsed on the host): no host-device
 * copies, asynchronous on the stream.  A zstd-framed h_data is decoded on
 * the host and taken as hh_hct3_decompress does (synchronous). */
int32_t hh_hct3_decompress_device(hh_context *ctx, const uint8_t *h_data, const uint8_t *d_data, size_t len,
                                  const uint64_t *shape, uint32_t rank, int32_t out_dtype, void *d_out,
                                  void *stream);

/* CompressiveSpectralDecoder::{add_essentials, add_detail, reconstruct}
 * (crates/haagenti/src/compressive.rs:438-752) for the V3 (HCT3, f16) and V2
 * (HCT2, f32) layouts: fragment 0 (frag_index[0] must be 0) holds
 * [magic][width][height][retain][essential][detail_per_frag][bitmap][values],
 * detail fragments [u16 idx][u16 total][u32 count][values]; fragments with
 * frag_index 0 after the first are ignored.  Errors as the reference
 * (HH_ERR_CORRUPTED_DATA with detail SIZE / BITMAP_COUNT / HEADER); the V1
 * index-array layout is HH_ERR_UNSUPPORTED.  Writes width * height elements
 * of out_dtype (HH_ERR_BUFFER_TOO_SMALL when out_cap is less).
 * Synchronous. */
int32_t hh_spectral_reconstruct(hh_context *ctx, const uint8_t *const *frags, const size_t *frag_lens,
                                const uint16_t *frag_index, uint32_t nfrags, int32_t out_dtype,
                                void *d_out, uint64_t out_cap, uint32_t *width, uint32_t *height,
                                hh_block_status *status, void *stream);

/* One tensor of the turbo pipeline's output file (crates/haagenti/src/
 * pipeline/turbo.rs:315-419): a zstd frame around a fragment container
 * ([u16 n] then {u16 index, u16 flags, u64 XXH3-64 of the data, u32 len,
 * data} per fragment, :378-387) of CompressiveSpectralEncoder fragments,
 * decoded with every fragment as hh_spectral_reconstruct does.  With verify,
 * each fragment's XXH3-64 (HoloFragment::new, holotensor.rs:283-292) is
 * checked first (HH_ERR_CHECKSUM_MISMATCH, status->position = fragment).
 * The reference writes these files but has no decoder for them outside its
 * examples (GpuDecompressor reads the other fragment layout); this is the
 * loader entry for them.  Synchronous. */
int32_t hh_turbo_tensor_decode(hh_context *ctx, const uint8_t *data, size_t len, int32_t verify,
                               int32_t out_dtype, void *d_out, uint64_t out_cap, uint32_t *width,
                               uint32_t *height, hh_block_status *status, void *stream);

/* GpuDctContext::idct_2d_gpu / idct_2d for a whole rows x cols matrix
 * (crates/haagenti-cuda/src/dct_gpu.rs:1163-1227, 1404-1412): orthonormal
 * 2-D DCT-III of the row-major f32 d_in into d_out (out_dtype).  Two routes
 * (HH_OPT_DCT_ROUTE), as the reference switches to idct_2d_fft above 4096
 * (dct_gpu.rs:1081,1714-1722): an FFT route -- each side a multiple of 64
 * whose half has no prime factor above 7 and is at most 20480; every row
 * transformed by Makhoul's construction over an f32 FFT in LDS, a
 * transpose, the same along the other side, a transpose back -- and two
 * split-f16 MFMA products against cached DCT bases for every other shape
 * (both ~1e-6 x RMS; the 16-bit outputs are the round-to-nearest-even of
 * the f32 result).  Asynchronous on the stream. */
int32_t hh_idct_2d(hh_context *ctx, const float *d_in, uint32_t rows, uint32_t cols, int32_t out_dtype,
                   void *d_out, void *stream);

/* GpuDctContext::dct_2d (dct_gpu.rs:1381-1389, dct_2d_fft above 4096;
 * used by the turbo encoder, crates/haagenti/src/pipeline/turbo.rs:351-369):
 * orthonormal 2-D DCT-II of a row-major f32 matrix (dct_2d, dct.rs:282-308),
 * on the same two routes as hh_idct_2d.  Asynchronous. */
int32_t hh_dct_2d(hh_context *ctx, const float *d_in, uint32_t rows, uint32_t cols, float *d_out,
                  void *stream);

/* zstd::decode_all (zstd crate 0.13.3 / libzstd; RFC 8878 frames) on the
 * host: every frame of in[0..in_len) decoded and concatenated into out.
 * *written receives the decoded size (also when it exceeds out_cap:
 * HH_ERR_BUFFER_TOO_SMALL); a malformed stream, a dictionary frame or a
 * window above 2^27 bytes is HH_ERR_CORRUPTED_DATA.  Content checksums are
 * verified. */
int32_t hh_zstd_decompress(const uint8_t *in, size_t in_len, uint8_t *out, size_t out_cap, size_t *written);
/* XXH64 (the zstd content checksum, RFC 8878 section 3.1.1). */
uint64_t hh_xxh64(const uint8_t *data, size_t len, uint64_t seed);

/* Bytes of CompressiveSpectralEncoder's fragments for a width x height
 * tensor (compressive.rs:94-238); *retain_count / *essential_count receive
 * the coefficient counts (either may be NULL). */
size_t hh_spectral_encoded_size(uint32_t width, uint32_t height, uint16_t num_fragments, float retention,
                                float essential_ratio, uint32_t *retain_count, uint32_t *essential_count);

/* CompressiveSpectralEncoder::encode_2d_from_dct (compressive.rs:240-340) on
 * the host: top retention of the coefficients by magnitude (stable sort),
 * fragment 0 and num_fragments - 1 detail fragments, concatenated into out;
 * fragment f is out[frag_offsets[f] .. frag_offsets[f + 1]). */
int32_t hh_spectral_encode_from_dct(const float *coeffs, uint32_t width, uint32_t height, uint16_t num_fragments,
                                    float retention, float essential_ratio, uint8_t *out, size_t out_cap,
                                    uint64_t *frag_offsets, size_t *written);

#ifdef __cplusplus
}
#endif
#endif /* HAAGENTI_HIP_H */
