// Host-side runtime of the streaming decode: page-locked staging buffers
// (PinnedBuffer), a device memory pool (MemoryPool) and the pipeline that
// overlaps host -> device copies with decoding (DecompressionPipeline).
//
//   PinnedBuffer            crates/haagenti-cuda/src/memory.rs:156-196
//   MemoryPool, PoolStats   memory.rs:200-360
//   DecompressionPipeline   crates/haagenti-cuda/src/pipeline.rs:35-289
//
// The reference's pipeline keeps every stage on the host clock (a device
// synchronize between stages, pipeline.rs:212-232) and its pinned buffer is
// an ordinary Vec (memory.rs:161-168).  Here the staging is hipHostMalloc
// memory, the copy stream and the compute stream are ordered by events
// only, and the host waits only when it must reuse a staging slot or when
// the caller asks for a result:
//
//   submit(l):  [host]    wait until slot l % S is free (unit l - S done),
//                         copy the unit's bytes into its pinned staging
//                         (parallel memcpy) unless they were written there
//               [copy]    wait consumed[s]; H2D staging -> d_in[s]; copied[s]
//               [compute] wait copied[s]; LZ4 blocks -> tile bytes; tile
//                         decode -> the caller's outputs; consumed[s];
//                         block records D2H; done[s]
//
// so the H2D of unit l + 1 runs under the decode of unit l.
#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <iterator>
#include <map>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hh_internal.hpp"

namespace {

using hh::from_hip;

constexpr size_t kAlign = 256;
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// A fixed set of host threads running one parallel memcpy at a time.
class CopyPool {
  public:
    explicit CopyPool(unsigned n) {
        for (unsigned i = 1; i < n; i++) workers_.emplace_back([this, i] { run(i); });
        n_ = n;
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }
    void copy(uint8_t *dst, const uint8_t *src, size_t n) {
        if (n < (4u << 20) || n_ == 1) {
            std::memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> l(mu_);
            dst_ = dst;
            src_ = src;
            len_ = n;
            pending_ = n_ - 1;
            gen_++;
        }
        cv_.notify_all();
        part(0);
        std::unique_lock<std::mutex> l(mu_);
        done_cv_.wait(l, [this] { return pending_ == 0; });
    }

  private:
    void part(unsigned i) {
        const size_t chunk = align_up((len_ + n_ - 1) / n_, 4096);
        const size_t a = std::min(len_, chunk * i), b = std::min(len_, a + chunk);
        if (b > a) std::memcpy(dst_ + a, src_ + a, b - a);
    }
    void run(unsigned i) {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            part(i);
            std::lock_guard<std::mutex> l(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }
    std::vector<std::thread> workers_;
    unsigned n_ = 1;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    bool stop_ = false;
    uint64_t gen_ = 0;
    unsigned pending_ = 0;
    uint8_t *dst_ = nullptr;
    const uint8_t *src_ = nullptr;
    size_t len_ = 0;
};

}  // namespace

// ---------------------------------------------------------------- pool

struct hh_pool {
    int device = 0;
    uint8_t *base = nullptr;
    size_t total = 0;
    std::mutex mu;
    std::map<size_t, size_t> free_;             // offset -> bytes, coalesced
    std::unordered_map<size_t, size_t> used_;   // offset -> bytes
    size_t allocated = 0;
};

// ---------------------------------------------------------------- pipeline

namespace {

struct Slot {
    uint8_t *h_stage = nullptr;        // pinned (or pageable) staging
    uint8_t *d_in = nullptr;           // device copy of the staging
    hh_block_status *d_status = nullptr;
    hh_block_status *h_status = nullptr;
    hipEvent_t h2d_start = nullptr, copied = nullptr, dec_start = nullptr, consumed = nullptr,
               done = nullptr;
    bool busy = false;                 // holds a unit not yet collected
    uint64_t ticket = 0;
    uint32_t nblocks = 0;
    // caller's block index of each staged block (empty: the same order)
    std::vector<uint32_t> order;
    uint64_t in_bytes = 0, lz4_bytes = 0, out_bytes = 0;
};

struct Result {
    int32_t code = HH_OK;
    int64_t failed_block = -1;
    hh_block_status status = {};
    hh_pipeline_times times = {};
    bool waited = false;
};

// Collected results are kept (for their times) until finish(); past this
// many, the ones already waited for are dropped.
constexpr size_t kKeepResults = 1u << 16;

}  // namespace

struct hh_pipeline {
    hh_context *ctx = nullptr;
    hh_pool *pool = nullptr;
    hh_pipeline_config cfg = {};
    hipStream_t copy = nullptr, compute = nullptr;
    std::vector<Slot> slots;
    uint8_t *d_tiles = nullptr;
    hipEvent_t t0 = nullptr;
    uint64_t next_ticket = 0;
    std::unordered_map<uint64_t, Result> results;   // collected, not yet waited for
    hh_pipeline_stats stats = {};
    CopyPool *copier = nullptr;
    std::vector<void *> device_allocs;
};

namespace {

int32_t dev_alloc(hh_pipeline *p, size_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0) bytes = kAlign;
    if (p->pool) return hh_pool_allocate(p->pool, bytes, 0, out);
    const hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) return from_hip(e);
    p->device_allocs.push_back(*out);
    return HH_OK;
}

void release(hh_pipeline *p) {
    for (Slot &s : p->slots) {
        for (hipEvent_t e : {s.h2d_start, s.copied, s.dec_start, s.consumed, s.done})
            if (e) (void)hipEventDestroy(e);
        if (s.h_stage) {
            if (p->cfg.use_pinned_memory)
                (void)hipHostFree(s.h_stage);
            else
                std::free(s.h_stage);
        }
        if (s.h_status) (void)hipHostFree(s.h_status);
        if (p->pool) {
            if (s.d_in) hh_pool_recycle(p->pool, s.d_in);
            if (s.d_status) hh_pool_recycle(p->pool, s.d_status);
        }
    }
    if (p->pool && p->d_tiles) hh_pool_recycle(p->pool, p->d_tiles);
    for (void *a : p->device_allocs) (void)hipFree(a);
    if (p->t0) (void)hipEventDestroy(p->t0);
    if (p->copy) (void)hipStreamDestroy(p->copy);
    if (p->compute) (void)hipStreamDestroy(p->compute);
    delete p->copier;
}

float ms_between(hipEvent_t a, hipEvent_t b) {
    float ms = 0.f;
    return hipEventElapsedTime(&ms, a, b) == hipSuccess ? ms : 0.f;
}

// Waits for the unit in slot s and records its result (statistics, first
// failing block, event times).
int32_t collect(hh_pipeline *p, Slot &s) {
    if (!s.busy) return HH_OK;
    const hipError_t e = hipEventSynchronize(s.done);
    if (e != hipSuccess) return from_hip(e);
    Result r;
    // the first failing block in the caller's order
    for (uint32_t b = 0; b < s.nblocks; b++) {
        const int64_t cb = s.order.empty() ? (int64_t)b : (int64_t)s.order[b];
        if (s.h_status[b].code != HH_OK && (r.failed_block < 0 || cb < r.failed_block)) {
            r.code = s.h_status[b].code;
            r.status = s.h_status[b];
            r.failed_block = cb;
            if (s.order.empty()) break;
        }
    }
    r.times.h2d_start_ms = ms_between(p->t0, s.h2d_start);
    r.times.h2d_end_ms = ms_between(p->t0, s.copied);
    r.times.decode_start_ms = ms_between(p->t0, s.dec_start);
    r.times.decode_end_ms = ms_between(p->t0, s.consumed);
    p->stats.units += 1;
    p->stats.blocks_processed += s.nblocks;
    p->stats.bytes_read += s.in_bytes;
    p->stats.bytes_decompressed += s.lz4_bytes;
    p->stats.bytes_output += s.out_bytes;
    p->stats.transfer_time_ns += (uint64_t)(1e6 * (r.times.h2d_end_ms - r.times.h2d_start_ms));
    p->stats.decompress_time_ns += (uint64_t)(1e6 * (r.times.decode_end_ms - r.times.decode_start_ms));
    if (p->results.size() >= kKeepResults)
        for (auto it = p->results.begin(); it != p->results.end();)
            it = it->second.waited ? p->results.erase(it) : std::next(it);
    p->results[s.ticket] = r;
    s.busy = false;
    return HH_OK;
}

size_t elem_bytes(int32_t dtype) { return dtype == HH_F32 ? 4 : 2; }

// Tensors of a unit that the fused launch decodes (hh_pipeline_submit with
// the tile scratch as LZ4 output).  Tensor i's tiles are packed at pos[i] of
// the LZ4 output; it qualifies when the blocks whose output lies in its
// tile bytes cut them into runs of tpb whole tiles in ascending output
// order (the last run the rest), each at most fused_block_max() bytes, and
// no block reaches into it from outside.  With HH_PIPE_AUTO only tensors
// with k >= 1024 are taken: sparser tiles compress into blocks of many short
// sequences, which the LZ4 launch decodes with more blocks in flight per CU
// than the fused launch's three LDS block buffers allow.  `order` lists the
// fused tensors' blocks first (tensor by tensor), then every other block in
// the caller's order.
struct FusedPlan {
    std::vector<uint32_t> fused;  // tensor indices
    std::vector<uint32_t> tpb;    // their tiles per block
    uint32_t nblocks = 0;         // their blocks: the first entries of `order`
    std::vector<uint32_t> order;  // staged block -> caller's block
};

FusedPlan plan_fused(int32_t route, const hh_hctt_tensor *tensors, uint32_t ntensors, const uint64_t *pos,
                     const uint64_t *out_off, const uint32_t *out_cap, uint32_t nblocks) {
    FusedPlan P;
    if (route == HH_PIPE_TWO_LAUNCH || ntensors == 0 || nblocks == 0) return P;
    std::vector<std::vector<uint32_t>> mine(ntensors);
    std::vector<char> ok(ntensors, 1);
    for (uint32_t b = 0; b < nblocks; b++) {
        const uint64_t lo = out_off[b], hi = lo + out_cap[b];
        // the tensors whose tile bytes [pos[i], pos[i + 1]) the block's
        // output range meets
        uint32_t i = (uint32_t)(std::upper_bound(pos, pos + ntensors + 1, lo) - pos);
        i = i > 0 ? i - 1 : 0;
        if (lo >= pos[ntensors]) continue;  // past every tensor
        if (hi <= pos[i + 1] && out_cap[b] > 0) {
            mine[i].push_back(b);
        } else {
            for (uint32_t j = i; j < ntensors && pos[j] < (hi > lo ? hi : lo + 1); j++) ok[j] = 0;
        }
    }
    const uint32_t fmax = hh::fused_block_max();
    std::vector<char> taken(nblocks, 0);
    for (uint32_t i = 0; i < ntensors; i++) {
        const hh_hctt_tensor &T = tensors[i];
        const uint64_t tb = hh_hctt_tile_bytes(T.k);
        const uint64_t nt = (uint64_t)(T.rows / 64) * (T.cols / 64);
        if (!ok[i] || nt == 0 || mine[i].empty() || T.tiles_len != nt * tb) continue;
        if (route == HH_PIPE_AUTO && T.k < 1024u) continue;
        std::vector<uint32_t> &m = mine[i];
        std::sort(m.begin(), m.end(), [&](uint32_t a, uint32_t c) { return out_off[a] < out_off[c]; });
        const uint64_t run = out_cap[m[0]];
        if (run % tb || run > fmax) continue;
        const uint64_t tpb = run / tb;
        if ((uint64_t)m.size() != (nt + tpb - 1) / tpb) continue;
        bool exact = true;
        for (size_t j = 0; j < m.size() && exact; j++) {
            const uint64_t want = j + 1 < m.size() ? run : (nt - j * tpb) * tb;
            exact = out_off[m[j]] == pos[i] + j * run && out_cap[m[j]] == want;
        }
        if (!exact) continue;
        P.fused.push_back(i);
        P.tpb.push_back((uint32_t)tpb);
        for (uint32_t b : m) {
            P.order.push_back(b);
            taken[b] = 1;
        }
    }
    if (P.fused.empty()) {
        P.order.clear();
        return P;
    }
    P.nblocks = (uint32_t)P.order.size();
    for (uint32_t b = 0; b < nblocks; b++)
        if (!taken[b]) P.order.push_back(b);
    return P;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- pinned

int32_t hh_pinned_alloc(size_t bytes, void **out) {
    if (!out) return HH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    if (bytes == 0) return HH_OK;
    return from_hip(hipHostMalloc(out, bytes, hipHostMallocDefault));
}

int32_t hh_pinned_free(void *ptr) { return ptr ? from_hip(hipHostFree(ptr)) : HH_OK; }

// ---------------------------------------------------------------- pool

int32_t hh_pool_create(hh_context *ctx, size_t total_size, hh_pool **out) {
    if (!ctx || !out) return HH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    hh::DeviceGuard guard(ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    hh_pool *p = new hh_pool();
    p->device = ctx->device;
    p->total = align_up(total_size, kAlign);
    if (p->total) {
        void *b = nullptr;
        const hipError_t e = hipMalloc(&b, p->total);
        if (e != hipSuccess) {
            delete p;
            return from_hip(e);
        }
        p->base = reinterpret_cast<uint8_t *>(b);
        p->free_[0] = p->total;
    }
    *out = p;
    return HH_OK;
}

void hh_pool_destroy(hh_pool *p) {
    if (!p) return;
    hh::DeviceGuard guard(p->device);
    if (p->base) (void)hipFree(p->base);
    delete p;
}

int32_t hh_pool_allocate(hh_pool *p, size_t size, int32_t zero, void **out) {
    if (!p || !out) return HH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    const size_t need = align_up(size ? size : 1, kAlign);
    size_t off = 0;
    {
        std::lock_guard<std::mutex> l(p->mu);
        auto it = p->free_.begin();
        for (; it != p->free_.end() && it->second < need; ++it) {
        }
        if (it == p->free_.end()) return HH_ERR_OUT_OF_MEMORY;  // OutOfMemory {requested, available}
        off = it->first;
        const size_t have = it->second;
        p->free_.erase(it);
        if (have > need) p->free_[off + need] = have - need;
        p->used_[off] = need;
        p->allocated += need;
    }
    *out = p->base + off;
    if (zero) {  // MemoryPool::allocate hands out zeroed buffers (alloc_zeros)
        hh::DeviceGuard guard(p->device);
        const hipError_t e = hipMemset(*out, 0, size);
        if (e != hipSuccess) {
            hh_pool_recycle(p, *out);
            *out = nullptr;
            return from_hip(e);
        }
    }
    return HH_OK;
}

int32_t hh_pool_recycle(hh_pool *p, void *ptr) {
    if (!p || !ptr) return HH_ERR_INVALID_ARGUMENT;
    const uint8_t *q = reinterpret_cast<const uint8_t *>(ptr);
    if (q < p->base || q >= p->base + p->total) return HH_ERR_INVALID_ARGUMENT;
    const size_t off = (size_t)(q - p->base);
    std::lock_guard<std::mutex> l(p->mu);
    auto u = p->used_.find(off);
    if (u == p->used_.end()) return HH_ERR_INVALID_ARGUMENT;
    size_t start = off, len = u->second;
    p->allocated -= len;
    p->used_.erase(u);
    auto next = p->free_.lower_bound(start);
    if (next != p->free_.end() && next->first == start + len) {  // merge with the extent after
        len += next->second;
        next = p->free_.erase(next);
    }
    if (next != p->free_.begin()) {  // and with the one before
        auto prev = std::prev(next);
        if (prev->first + prev->second == start) {
            start = prev->first;
            len += prev->second;
            p->free_.erase(prev);
        }
    }
    p->free_[start] = len;
    return HH_OK;
}

int32_t hh_pool_get_stats(hh_pool *p, hh_pool_stats *out) {
    if (!p || !out) return HH_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> l(p->mu);
    out->total_size = p->total;
    out->allocated = p->allocated;
    out->available = p->total - p->allocated;
    out->free_buffers = p->free_.size();
    size_t fb = 0, largest = 0;
    for (const auto &f : p->free_) {
        fb += f.second;
        largest = std::max(largest, f.second);
    }
    out->free_buffer_bytes = fb;
    out->largest_free = largest;
    return HH_OK;
}

// ---------------------------------------------------------------- pipeline

void hh_pipeline_default_config(hh_pipeline_config *cfg) {
    if (!cfg) return;
    std::memset(cfg, 0, sizeof(*cfg));
    cfg->num_staging_buffers = 2;
    cfg->staging_buffer_size = 4ull << 20;  // PipelineConfig::default (pipeline.rs:51-59)
    cfg->max_blocks = 65536;
    cfg->tile_scratch_size = 0;
    cfg->use_pinned_memory = 1;
    cfg->copy_threads = 8;
}

int32_t hh_pipeline_create(hh_context *ctx, hh_pool *pool, const hh_pipeline_config *cfg, hh_pipeline **out) {
    if (!ctx || !cfg || !out) return HH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    if (cfg->num_staging_buffers < 1 || cfg->num_staging_buffers > 16 || cfg->max_blocks < 1 ||
        cfg->staging_buffer_size < 64)
        return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    hh_pipeline *p = new hh_pipeline();
    p->ctx = ctx;
    p->pool = pool;
    p->cfg = *cfg;
    p->cfg.staging_buffer_size = align_up(cfg->staging_buffer_size, kAlign);
    int32_t rc = HH_OK;
    hipError_t e = hipStreamCreateWithFlags(&p->copy, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->compute, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&p->t0);
    if (e != hipSuccess) rc = from_hip(e);
    p->slots.resize(cfg->num_staging_buffers);
    for (Slot &s : p->slots) {
        if (rc != HH_OK) break;
        const size_t sb = p->cfg.staging_buffer_size;
        if (p->cfg.use_pinned_memory) {
            e = hipHostMalloc(reinterpret_cast<void **>(&s.h_stage), sb, hipHostMallocDefault);
            if (e != hipSuccess) rc = from_hip(e);
        } else {
            s.h_stage = reinterpret_cast<uint8_t *>(std::malloc(sb));
            if (!s.h_stage) rc = HH_ERR_OUT_OF_MEMORY;
        }
        if (rc == HH_OK) {
            e = hipHostMalloc(reinterpret_cast<void **>(&s.h_status), sizeof(hh_block_status) * cfg->max_blocks,
                              hipHostMallocDefault);
            if (e != hipSuccess) rc = from_hip(e);
        }
        void *d = nullptr;
        if (rc == HH_OK) rc = dev_alloc(p, sb, &d);
        s.d_in = reinterpret_cast<uint8_t *>(d);
        if (rc == HH_OK) rc = dev_alloc(p, sizeof(hh_block_status) * cfg->max_blocks, &d);
        s.d_status = reinterpret_cast<hh_block_status *>(d);
        for (hipEvent_t *ev : {&s.h2d_start, &s.copied, &s.dec_start, &s.consumed, &s.done})
            if (rc == HH_OK) {
                e = hipEventCreate(ev);
                if (e != hipSuccess) rc = from_hip(e);
            }
    }
    if (rc == HH_OK && cfg->tile_scratch_size) {
        void *d = nullptr;
        rc = dev_alloc(p, cfg->tile_scratch_size, &d);
        p->d_tiles = reinterpret_cast<uint8_t *>(d);
    }
    if (rc == HH_OK) {
        // every event starts out recorded, so the first waits on them pass
        e = hipEventRecord(p->t0, p->compute);
        for (Slot &s : p->slots)
            for (hipEvent_t ev : {s.h2d_start, s.copied, s.dec_start, s.consumed, s.done})
                if (e == hipSuccess) e = hipEventRecord(ev, p->compute);
        if (e == hipSuccess) e = hipStreamSynchronize(p->compute);
        if (e != hipSuccess) rc = from_hip(e);
    }
    if (rc != HH_OK) {
        release(p);
        delete p;
        return rc;
    }
    p->copier = new CopyPool(cfg->copy_threads ? cfg->copy_threads : 8);
    *out = p;
    return HH_OK;
}

void hh_pipeline_destroy(hh_pipeline *p) {
    if (!p) return;
    hh::DeviceGuard guard(p->ctx->device);
    if (p->copy) (void)hipStreamSynchronize(p->copy);
    if (p->compute) (void)hipStreamSynchronize(p->compute);
    release(p);
    delete p;
}

int32_t hh_pipeline_streams(hh_pipeline *p, void **copy_stream, void **compute_stream) {
    if (!p) return HH_ERR_INVALID_ARGUMENT;
    if (copy_stream) *copy_stream = p->copy;
    if (compute_stream) *compute_stream = p->compute;
    return HH_OK;
}

int32_t hh_pipeline_next_staging(hh_pipeline *p, uint8_t **h_ptr, size_t *cap) {
    if (!p || !h_ptr) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    Slot &s = p->slots[p->next_ticket % p->slots.size()];
    const int32_t rc = collect(p, s);  // the slot's previous unit must be done with it
    if (rc != HH_OK) return rc;
    *h_ptr = s.h_stage;
    if (cap) *cap = p->cfg.staging_buffer_size;
    return HH_OK;
}

int32_t hh_pipeline_submit(hh_pipeline *p, const uint8_t *h_data, size_t len, const uint64_t *h_in_off,
                           const uint32_t *h_in_len, const uint64_t *h_out_off, const uint32_t *h_out_cap,
                           uint32_t nblocks, uint8_t *d_lz4_out, uint64_t lz4_out_cap, const hh_hctt_tensor *tensors,
                           uint32_t ntensors, int32_t out_dtype, void *after_event, uint64_t *ticket) {
    if (!p || (!h_data && len) || (!tensors && ntensors)) return HH_ERR_INVALID_ARGUMENT;
    if (nblocks && (!h_in_off || !h_in_len || !h_out_off || !h_out_cap)) return HH_ERR_INVALID_ARGUMENT;
    if (nblocks > p->cfg.max_blocks) return HH_ERR_BUFFER_TOO_SMALL;
    if (ntensors && out_dtype != HH_F32 && out_dtype != HH_F16 && out_dtype != HH_BF16) return HH_ERR_UNSUPPORTED;
    // layout of a staged unit: [data][in_off u64][out_off u64][in_len u32][out_cap u32]
    const size_t tab = align_up(len, 16);
    const size_t bytes = tab + (size_t)nblocks * 24;
    if (bytes > p->cfg.staging_buffer_size) return HH_ERR_BUFFER_TOO_SMALL;
    // where the LZ4 output goes: the caller's buffer, or the tile scratch
    // where the tensors' tiles are packed in order
    uint8_t *lz4_out = d_lz4_out;
    uint64_t lz4_cap = lz4_out_cap;
    if (!lz4_out) {
        lz4_out = p->d_tiles;
        lz4_cap = p->d_tiles ? p->cfg.tile_scratch_size : 0;
    }
    uint64_t tiles_total = 0, out_bytes = 0, ntiles_total = 0;
    for (uint32_t i = 0; i < ntensors; i++) {
        if (tensors[i].d_tiles != nullptr) return HH_ERR_INVALID_ARGUMENT;
        if (tensors[i].tiles_len > lz4_cap - tiles_total) return HH_ERR_BUFFER_TOO_SMALL;
        // the tile decode's own checks, made before anything is enqueued
        // (its d_tiles points into the LZ4 output once enqueued)
        hh_hctt_tensor t = tensors[i];
        t.d_tiles = lz4_out ? lz4_out + tiles_total : nullptr;
        size_t nt = 0;
        const int32_t trc = hh::check_hctt_tensor(t, &nt);
        if (trc != HH_OK) return trc;
        ntiles_total += nt;
        tiles_total += tensors[i].tiles_len;
        out_bytes += (uint64_t)tensors[i].rows * tensors[i].cols * elem_bytes(out_dtype);
    }
    if (ntiles_total > 0xffffffffull) return HH_ERR_UNSUPPORTED;
    if (nblocks && !lz4_out) return HH_ERR_INVALID_ARGUMENT;
    // the tensors' packed tile offsets in the LZ4 output, and which of them
    // the fused launch takes (only when that output is the tile scratch)
    std::vector<uint64_t> pos(ntensors + 1, 0);
    for (uint32_t i = 0; i < ntensors; i++) pos[i + 1] = pos[i] + tensors[i].tiles_len;
    const FusedPlan plan = d_lz4_out ? FusedPlan{}
                                     : plan_fused(p->ctx->pipeline_route, tensors, ntensors, pos.data(), h_out_off,
                                                  h_out_cap, nblocks);
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    Slot &s = p->slots[p->next_ticket % p->slots.size()];
    int32_t rc = collect(p, s);
    if (rc != HH_OK) return rc;
    // stage the unit: no host copy when the caller wrote it in place, or
    // when it already sits in page-locked memory (copied to the device from
    // there; the caller keeps it unchanged until the unit is waited for)
    bool direct = false;
    if (h_data != s.h_stage && len) {
        for (const Slot &o : p->slots)
            if (h_data >= o.h_stage && h_data < o.h_stage + p->cfg.staging_buffer_size)
                return HH_ERR_INVALID_ARGUMENT;  // another slot's staging
        hipPointerAttribute_t attr;
        if (hipPointerGetAttributes(&attr, h_data) == hipSuccess && attr.type == hipMemoryTypeHost)
            direct = true;
        else
            (void)hipGetLastError();  // pageable memory: clear the lookup's error
        if (!direct) p->copier->copy(s.h_stage, h_data, len);
    }
    uint64_t lz4_bytes = 0;
    if (nblocks && plan.order.empty()) {
        std::memcpy(s.h_stage + tab, h_in_off, 8 * (size_t)nblocks);
        std::memcpy(s.h_stage + tab + 8 * (size_t)nblocks, h_out_off, 8 * (size_t)nblocks);
        std::memcpy(s.h_stage + tab + 16 * (size_t)nblocks, h_in_len, 4 * (size_t)nblocks);
        std::memcpy(s.h_stage + tab + 20 * (size_t)nblocks, h_out_cap, 4 * (size_t)nblocks);
    } else if (nblocks) {
        // the fused tensors' blocks first (plan order)
        uint64_t *io = reinterpret_cast<uint64_t *>(s.h_stage + tab);
        uint64_t *oo = io + nblocks;
        uint32_t *il = reinterpret_cast<uint32_t *>(oo + nblocks);
        uint32_t *oc = il + nblocks;
        for (uint32_t j = 0; j < nblocks; j++) {
            const uint32_t b = plan.order[j];
            io[j] = h_in_off[b];
            oo[j] = h_out_off[b];
            il[j] = h_in_len[b];
            oc[j] = h_out_cap[b];
        }
    }
    for (uint32_t b = 0; b < nblocks; b++) lz4_bytes += h_out_cap[b];
    s.order = plan.order;
    // copy stream: H2D once the device slot's previous decode is done
    hipError_t e = hipStreamWaitEvent(p->copy, s.consumed, 0);
    if (e == hipSuccess) e = hipEventRecord(s.h2d_start, p->copy);
    if (direct) {
        if (e == hipSuccess) e = hipMemcpyAsync(s.d_in, h_data, len, hipMemcpyHostToDevice, p->copy);
        if (e == hipSuccess && bytes > tab)
            e = hipMemcpyAsync(s.d_in + tab, s.h_stage + tab, bytes - tab, hipMemcpyHostToDevice, p->copy);
    } else if (e == hipSuccess && bytes) {
        e = hipMemcpyAsync(s.d_in, s.h_stage, bytes, hipMemcpyHostToDevice, p->copy);
    }
    if (e == hipSuccess) e = hipEventRecord(s.copied, p->copy);
    // compute stream: decode once the copy has landed
    if (e == hipSuccess) e = hipStreamWaitEvent(p->compute, s.copied, 0);
    if (e == hipSuccess && after_event)
        e = hipStreamWaitEvent(p->compute, reinterpret_cast<hipEvent_t>(after_event), 0);
    if (e == hipSuccess) e = hipEventRecord(s.dec_start, p->compute);
    if (e != hipSuccess) return from_hip(e);
    // the tensors the two launches decode
    std::vector<hh_hctt_tensor> rest, fused;
    {
        std::vector<char> is_fused(ntensors, 0);
        for (uint32_t i : plan.fused) is_fused[i] = 1;
        for (uint32_t i = 0; i < ntensors; i++) {
            hh_hctt_tensor t = tensors[i];
            t.d_tiles = lz4_out + pos[i];
            (is_fused[i] ? fused : rest).push_back(t);
        }
    }
    const uint8_t *t = s.d_in + tab;
    const uint64_t *d_in_off = reinterpret_cast<const uint64_t *>(t);
    const uint64_t *d_out_off = reinterpret_cast<const uint64_t *>(t + 8 * (size_t)nblocks);
    const uint32_t *d_in_len = reinterpret_cast<const uint32_t *>(t + 16 * (size_t)nblocks);
    const uint32_t *d_out_cap = reinterpret_cast<const uint32_t *>(t + 20 * (size_t)nblocks);
    // fused launch first: the LZ4 launch's long sequence chains then overlap
    // its last workgroups
    if (plan.nblocks) {
        e = hh::launch_hctt_lz4_fused(
            fused.data(), (uint32_t)fused.size(), plan.tpb.data(), s.d_in, len, d_in_off, d_in_len, s.d_status,
            out_dtype, p->ctx->d_basis, p->ctx->num_cus, p->ctx->fused_poll_limit,
            hh::lz4_decoder_for_tiles(p->ctx, fused.data(), (uint32_t)fused.size()) == HH_LZ4_SEQ, p->compute);
        if (e != hipSuccess) return from_hip(e);
    }
    const uint32_t nb2 = nblocks - plan.nblocks;
    if (nb2) {
        const uint32_t f = plan.nblocks;
        // the tile scratch: a short block's tail zeroed, as in the fused launch
        const hh::Lz4Batch B = {s.d_in, len, d_in_off + f, d_in_len + f, lz4_out,
                                d_lz4_out ? lz4_cap : tiles_total, d_out_off + f, d_out_cap + f, nb2,
                                s.d_status + f, d_lz4_out ? 0u : 1u};
        e = hh::launch_lz4_batch(B, hh::lz4_decoder_for_tiles(p->ctx, rest.data(), (uint32_t)rest.size()),
                                 p->compute);
        if (e != hipSuccess) return from_hip(e);
    }
    for (size_t i = 0; i < rest.size(); i += 8) {
        const uint32_t n = rest.size() - i < 8 ? (uint32_t)(rest.size() - i) : 8u;
        rc = hh_hctt_decode_batch(p->ctx, rest.data() + i, n, out_dtype, p->compute);
        if (rc != HH_OK) return rc;
    }
    e = hipEventRecord(s.consumed, p->compute);
    if (e == hipSuccess && nblocks)
        e = hipMemcpyAsync(s.h_status, s.d_status, sizeof(hh_block_status) * nblocks, hipMemcpyDeviceToHost,
                           p->compute);
    if (e == hipSuccess) e = hipEventRecord(s.done, p->compute);
    if (e != hipSuccess) return from_hip(e);
    s.busy = true;
    s.ticket = p->next_ticket;
    s.nblocks = nblocks;
    s.in_bytes = len;
    s.lz4_bytes = lz4_bytes;
    s.out_bytes = out_bytes;
    if (ticket) *ticket = p->next_ticket;
    p->next_ticket++;
    return HH_OK;
}

int32_t hh_pipeline_wait(hh_pipeline *p, uint64_t ticket, hh_block_status *status, int64_t *failed_block) {
    if (failed_block) *failed_block = -1;
    if (status) std::memset(status, 0, sizeof(*status));
    if (!p || ticket >= p->next_ticket) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    Slot &s = p->slots[ticket % p->slots.size()];
    if (s.busy && s.ticket == ticket) {
        const int32_t rc = collect(p, s);
        if (rc != HH_OK) return rc;
    }
    auto it = p->results.find(ticket);
    if (it == p->results.end() || it->second.waited) return HH_ERR_INVALID_ARGUMENT;  // already waited for
    it->second.waited = true;
    const Result r = it->second;
    if (status) *status = r.status;
    if (failed_block) *failed_block = r.failed_block;
    return r.code;
}

int32_t hh_pipeline_get_times(hh_pipeline *p, uint64_t ticket, hh_pipeline_times *out) {
    if (!p || !out || ticket >= p->next_ticket) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    Slot &s = p->slots[ticket % p->slots.size()];
    if (s.busy && s.ticket == ticket) {
        const int32_t rc = collect(p, s);
        if (rc != HH_OK) return rc;
    }
    auto it = p->results.find(ticket);
    if (it == p->results.end()) return HH_ERR_INVALID_ARGUMENT;
    *out = it->second.times;
    return HH_OK;
}

int32_t hh_pipeline_stream_wait(hh_pipeline *p, uint64_t ticket, void *stream) {
    if (!p || ticket >= p->next_ticket) return HH_ERR_INVALID_ARGUMENT;
    const Slot &s = p->slots[ticket % p->slots.size()];
    if (!(s.busy && s.ticket == ticket)) return HH_OK;  // already complete
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    return from_hip(hipStreamWaitEvent(reinterpret_cast<hipStream_t>(stream), s.consumed, 0));
}

int32_t hh_pipeline_finish(hh_pipeline *p, hh_block_status *status, int64_t *failed_block, uint64_t *failed_ticket) {
    if (failed_block) *failed_block = -1;
    if (failed_ticket) *failed_ticket = UINT64_MAX;
    if (status) std::memset(status, 0, sizeof(*status));
    if (!p) return HH_ERR_INVALID_ARGUMENT;
    hh::DeviceGuard guard(p->ctx->device);
    if (guard.status() != hipSuccess) return from_hip(guard.status());
    for (Slot &s : p->slots) {
        const int32_t rc = collect(p, s);
        if (rc != HH_OK) return rc;
    }
    // the first failure among the units not waited for, then forget them
    int32_t code = HH_OK;
    uint64_t first = UINT64_MAX;
    for (const auto &kv : p->results)
        if (!kv.second.waited && kv.second.code != HH_OK && kv.first < first) {
            first = kv.first;
            code = kv.second.code;
            if (status) *status = kv.second.status;
            if (failed_block) *failed_block = kv.second.failed_block;
        }
    if (failed_ticket) *failed_ticket = first;
    p->results.clear();
    return code;
}

int32_t hh_pipeline_get_stats(hh_pipeline *p, hh_pipeline_stats *out) {
    if (!p || !out) return HH_ERR_INVALID_ARGUMENT;
    *out = p->stats;
    return HH_OK;
}

void hh_pipeline_reset_stats(hh_pipeline *p) {
    if (p) std::memset(&p->stats, 0, sizeof(p->stats));
}

}  // extern "C"
