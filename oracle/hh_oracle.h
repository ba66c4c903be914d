/*
 * hh_oracle.h -- CPU restatement of the reference HCT decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product (haagenti_amd) never links or calls it.
 *
 * Every function restates a reference function (cited as file:line, paths
 * relative to the reference repository root) in plain C11 so that the GPU
 * path can be compared with it on identical inputs.
 *
 * Parity status of each function (how the restatement itself is pinned) is
 * listed next to it; tests/test_oracle_*.py hold the checks.
 */
#ifndef HH_ORACLE_H
#define HH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error kinds, same meaning as haagenti_core::Error
 * (crates/haagenti-core/src/error.rs:10-60). */
enum {
    HHO_OK = 0,
    HHO_CORRUPTED_DATA = 1,
    HHO_BUFFER_TOO_SMALL = 2,
    HHO_UNEXPECTED_EOF = 3,
    HHO_UNSUPPORTED = 5, /* Error::Unsupported */
    HHO_ALGORITHM = 6,   /* Error::Algorithm ("hct" read failures, tensor.rs:421-431,470-480) */
    HHO_INVALID_DATA = 7, /* CudaError::InvalidData (crates/haagenti-cuda/src/error.rs) */
};

/* Sub-kinds of CorruptedData raised by decompress_block / the HCT parsers. */
enum {
    HHO_CORRUPT_NONE = 0,
    HHO_CORRUPT_ZERO_OFFSET = 1,      /* block.rs:320-322 "invalid zero offset" */
    HHO_CORRUPT_OFFSET_BEYOND = 2,    /* block.rs:323-325 "offset beyond output at offset N" */
    HHO_CORRUPT_BITMAP_COUNT = 3,     /* compressive.rs:630-636 popcount != k */
    HHO_CORRUPT_HEADER = 4,           /* tensor.rs:311-331 magic/version/algo/dtype */
    HHO_CORRUPT_SIZE = 5,             /* size/shape inconsistencies in containers */
    HHO_CORRUPT_HEADER_CHECKSUM = 6,  /* tensor.rs:857-865 "header checksum mismatch" */
    HHO_CORRUPT_BLOCK_CHECKSUM = 7,   /* tensor.rs:965-974 "block N checksum mismatch" */
    HHO_CORRUPT_QUANT_SCHEME = 8,     /* tensor.rs:158-173 "unknown quantization scheme" */
};

typedef struct hho_err {
    int32_t kind;       /* HHO_* */
    int32_t sub;        /* HHO_CORRUPT_* */
    uint64_t position;  /* UnexpectedEof: bytes_read; OffsetBeyond: output_pos */
    uint64_t required;  /* BufferTooSmall: required */
    uint64_t provided;  /* BufferTooSmall: provided */
} hho_err;

/* ---------------- LZ4 raw block (crates/haagenti-lz4/src/block.rs) ------- */

/* block.rs:370-373 */
size_t hho_lz4_max_compressed_size(size_t input_len);

/* block.rs:73-147 (+ write_sequence :150-209, write_last_literals :212-251).
 * Returns HHO_OK and sets *written, or HHO_BUFFER_TOO_SMALL. */
int hho_lz4_compress_block(const uint8_t *in, size_t in_len, uint8_t *out,
                           size_t out_cap, size_t *written, hho_err *err);

/* block.rs:261-366.  out_len is output.len(), output_size the expected size
 * (they are equal in every reference caller, decompress.rs:59-68). */
int hho_lz4_decompress_block(const uint8_t *in, size_t in_len, uint8_t *out,
                             size_t out_len, size_t output_size,
                             size_t *written, hho_err *err);

/* Many independent blocks; nthreads workers (0 = all cores).  Per-block
 * status in kinds[]/written[].  Mirrors the rayon par_iter structure of
 * crates/haagenti/src/pipeline/turbo.rs:236-261 for the CPU baseline. */
void hho_lz4_decompress_batch(const uint8_t *in, const uint64_t *in_off,
                              const uint32_t *in_len, uint8_t *out,
                              const uint64_t *out_off, const uint32_t *out_cap,
                              size_t nblocks, int32_t *kinds, uint64_t *written,
                              int nthreads);

/* ---------------- INT4 (crates/haagenti/src/testing/quantization.rs) ------ */

uint16_t hho_f32_to_f16_bits(float v);          /* :136-163 (truncating) */
float hho_f16_bits_to_f32(uint16_t h);          /* :166-197 */
/* Same over an array, returning raw f32 bit patterns (keeps NaN payloads). */
void hho_f16_bits_to_f32_bits(const uint16_t *h, size_t n, uint32_t *out);
size_t hho_int4_compressed_size(size_t n);      /* :202-210 */
/* :30-70; returns bytes written (== hho_int4_compressed_size(n)). */
size_t hho_quantize_int4(const float *w, size_t n, uint8_t *out);
/* :82-131; returns the number of elements produced (may be < n). */
size_t hho_dequantize_int4(const uint8_t *data, size_t data_len, size_t n,
                           float *out);
/* Same arithmetic over [begin, end) 32-element groups, threaded. */
size_t hho_dequantize_int4_mt(const uint8_t *data, size_t data_len, size_t n,
                              float *out, int nthreads);

/* ---------------- DCT (crates/haagenti-core/src/dct.rs) ------------------- */

void hho_dct_1d(const float *in, float *out, size_t n);        /* :79-129 */
void hho_dct_1d_direct(const float *in, float *out, size_t n); /* :133-146 */
void hho_idct_1d(const float *in, float *out, size_t n);       /* :154-259 */
void hho_idct_1d_direct(const float *in, float *out, size_t n);/* :263-277 */
void hho_dct_2d(const float *in, float *out, size_t width, size_t height);  /* :282-308 */
void hho_idct_2d(const float *in, float *out, size_t width, size_t height); /* :311-337 */
/* hho_idct_2d on nthreads threads (0: all cores), bit-identical. */
void hho_idct_2d_mt(const float *in, float *out, size_t width, size_t height, int nthreads);
void hho_dct_1d_f64(const double *in, double *out, size_t n);  /* :342-361 */
void hho_idct_1d_f64(const double *in, double *out, size_t n); /* :364-383 */
void hho_dct_2d_f64(const double *in, double *out, size_t w, size_t h);  /* :386-412 */
void hho_idct_2d_f64(const double *in, double *out, size_t w, size_t h); /* :415-441 */
/* crates/haagenti/src/hct_test_vectors.rs:43-75 and :78-107 */
void hho_reference_dct_2d(const float *in, float *out, size_t rows, size_t cols);
void hho_reference_idct_2d(const float *in, float *out, size_t rows, size_t cols);

/* ---------------- Spectral retention (crates/haagenti/src/compressive.rs) - */

/* k = max(1, (n as f32 * clamp(rho, .05, 1)) as usize)   (:97, :152) */
size_t hho_retain_count(size_t n, float rho);
/* Top-k by |c| (stable descending sort, :144-149), LSB-first bitmap of the
 * kept raster indices (:157-163); ascending kept indices into idx (:167-172).
 * NaN magnitudes sort last (the reference's order with NaN depends on its
 * sort algorithm; the decode path never sees it). */
void hho_topk_bitmap(const float *c, size_t n, size_t k, uint8_t *bitmap,
                     uint32_t *idx);
/* Bitmap -> ascending index map (:620-627). Returns the number of set bits. */
size_t hho_bitmap_index_map(const uint8_t *bitmap, size_t n, uint32_t *idx);

/* ---------------- HCT-T tile format (64x64 tiles, INT4 coefficients) ------ */
/* Tile bytes: [bitmap 512][ceil(k/32) f16 scales][ceil(k/2) nibble bytes]   */

size_t hho_hctt_tile_bytes(size_t k);
/* Encode one 64x64 tile: dct_2d -> top-k -> bitmap -> quantize_int4. */
void hho_hctt_encode_tile(const float *tile, size_t k, uint8_t *out);
/* Decode one tile: dequantize_int4 -> bitmap scatter -> idct_2d (f32).
 * Returns HHO_OK or HHO_CORRUPTED_DATA (bitmap popcount != k). */
int hho_hctt_decode_tile(const uint8_t *tile_bytes, size_t k, float *out64x64);
/* Same but the IDCT in f64 (truth), output f64. */
int hho_hctt_decode_tile_f64(const uint8_t *tile_bytes, size_t k, double *out);
/* Whole row-major rows x cols tensor (multiples of 64), tiles in row-major
 * tile order; threaded.  Output row-major f32. */
void hho_hctt_encode_tensor(const float *w, size_t rows, size_t cols, size_t k,
                            uint8_t *out, int nthreads);
int hho_hctt_decode_tensor(const uint8_t *tiles, size_t rows, size_t cols,
                           size_t k, float *out, int nthreads);

/* ---------------- HCT container (crates/haagenti-hct/src/tensor.rs) ------ */

/* Size of the v1 file HctWriter::finish writes for the given blocks. */
size_t hho_hct_file_size(size_t nblocks, size_t total_compressed);
/* HctWriter::compress_data + finish (:556-616) with the LZ4 compressor:
 * chunks data by block_size, compresses each chunk, writes header + index +
 * data into out (capacity out_cap).  Returns bytes written or 0 on error. */
size_t hho_hct_write_lz4(const uint8_t *data, size_t len, uint32_t block_size,
                         uint8_t dtype, const uint64_t *shape, int rank,
                         uint8_t *out, size_t out_cap);
/* HctReader::new + decompress_all (:417-515).  Writes the concatenated
 * output into out (capacity out_cap) and *written. */
int hho_hct_read_all_lz4(const uint8_t *file, size_t file_len, uint8_t *out,
                         size_t out_cap, size_t *written, hho_err *err);

/* ---------------- XXH3-64 (xxhash-rust 0.8.15 xxh3_64, seed 0) ----------
 * Call sites: tensor.rs:729,794,858,967.  Restated from the published XXH3
 * algorithm (xxHash 0.8: default 192-byte secret, 0-16 / 17-128 / 129-240 /
 * long-input paths); pinned against the xxhash library's outputs. */
uint64_t hho_xxh3_64(const uint8_t *data, size_t len);
/* The same over n buffers data[off[i], off[i] + len[i]) on nthreads threads. */
void hho_xxh3_64_batch(const uint8_t *data, const uint64_t *off, const uint32_t *len, size_t n,
                       uint64_t *out, int nthreads);

/* ---------------- HCT v2 container (tensor.rs:45-271, 676-1021) ---------- */

#define HHO_FLAG_HEADER_CHECKSUM 0x0001u
#define HHO_FLAG_BLOCK_CHECKSUMS 0x0002u
#define HHO_FLAG_QUANTIZATION 0x0004u

/* HctWriterV2 (:679-829) with the LZ4 compressor: flags as given (the
 * writer's default is HEADER_CHECKSUM | BLOCK_CHECKSUMS); quant8 is the
 * 8-byte QuantizationMetadata (:195-226) written when flags has
 * QUANTIZATION.  Returns bytes written or 0 on error. */
size_t hho_hct_write_v2_lz4(const uint8_t *data, size_t len, uint32_t block_size,
                            uint8_t dtype, const uint64_t *shape, int rank, uint16_t flags,
                            const uint8_t *quant8, uint8_t *out, size_t out_cap);
/* HctReaderV2::new + decompress_all_validated (:840-1012).  *failed_block
 * receives the index of the failing block, or -1 when the header stage fails. */
int hho_hct_read_all_v2_lz4(const uint8_t *file, size_t file_len, uint8_t *out,
                            size_t out_cap, size_t *written, hho_err *err,
                            int64_t *failed_block);
/* HctReaderV2::new + validate_checksums (:1014-1020). */
int hho_hct_validate_v2(const uint8_t *file, size_t file_len, hho_err *err,
                        int64_t *failed_block);

/* ---------------- HCT3 whole-tensor spectral ------------------------------
 * Fragment container of GpuDecompressor (crates/haagenti-cuda/src/
 * decompress.rs:322-427) and CompressiveSpectral{Encoder,Decoder}
 * (crates/haagenti/src/compressive.rs:67-752).  Parity: the coefficient
 * scatter is pinned bit-exactly against the reference's own C decoder
 * (ref/c/hct_decoder.h: hct_decode == hct_idct_2d of these coefficients,
 * built into oracle/_ref) on well-formed containers; the encoder and
 * decoder against each other (round trips, the reference's own MSE bounds,
 * compressive.rs:777-980) and the f16 rounding against numpy (IEEE RNE). */
uint16_t hho_f32_to_f16_rne(float v);
int hho_hct3_coefficients(const uint8_t *data, size_t len, size_t total, float *dense);
int hho_hct3_decode(const uint8_t *data, size_t len, const uint64_t *shape, size_t rank, float *out);
size_t hho_spectral_encode_from_dct(const float *dct, uint32_t width, uint32_t height, uint16_t nfrag,
                                    float retention, float essential_ratio, uint8_t *out, size_t cap,
                                    uint64_t *offsets);
int hho_spectral_reconstruct(const uint8_t *const *frags, const size_t *lens, const uint16_t *fidx, uint32_t nf,
                             float *out, size_t out_cap, uint32_t *width, uint32_t *height, hho_err *err);

#ifdef __cplusplus
}
#endif
#endif
