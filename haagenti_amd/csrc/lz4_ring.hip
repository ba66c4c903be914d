// Batched raw-LZ4 block decoder that keeps each block's recent output in
// LDS: one wavefront per block (the decoder itself is in lz4_ring.hpp).
#include "lz4_ring.hpp"

namespace hh {
namespace {

template <uint32_t R, uint32_t S>
__global__ __launch_bounds__(64) void lz4_ring_kernel(Lz4Batch B) {
    using D = ring::RingDec<R, S>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.x;
    if (b >= B.nblocks) return;

    int32_t code = HH_OK, detail = HH_CORRUPT_NONE;
    uint64_t pos = 0, req = 0;

    const uint64_t ioff = B.in_off[b];
    const uint32_t ilen = B.in_len[b];
    const uint64_t oofs = B.out_off[b];
    const uint32_t ocap = B.out_cap[b];
    const bool out_ok = oofs <= B.out_total && (uint64_t)ocap <= B.out_total - oofs;
    uint8_t *out = B.out + oofs;
    D d;
    d.ring = smem;
    d.stage = smem + R + D::kSFront;
    d.gbuf = B.in;
    d.gsz = B.in_total;
    d.ioff = ioff;
    d.a0 = (uint32_t)((uintptr_t)out & 15u);
    d.obase = out - d.a0;
    d.cap = ocap;
    d.sb = 0;
    d.at_end = false;
    d.wso = ring::kNoWin;
    d.w = 0;
    d.op = 0;
    d.fl = 0;
    d.lane = lane;

    if (ioff > B.in_total || (uint64_t)ilen > B.in_total - ioff || !out_ok) {
        code = HH_ERR_INVALID_ARGUMENT;
    } else {
        ring::parse_block(d, ilen, code, detail, pos, req);
        if (code == HH_OK) d.flush(true);
    }
    // a failed block's output reads as zeros (the reference returns no output)
    if (code != HH_OK && out_ok) {
        d.mem_sync();
        wave_zero_fill(out, d.cap, lane);
    } else if (code == HH_OK && B.zero_tail && d.op < d.cap) {
        wave_zero_fill(out + d.op, d.cap - d.op, lane);
    }
    if (lane == 0) {
        hh_block_status st;
        st.code = code;
        st.detail = detail;
        st.position = pos;
        st.required = req;
        st.written = code == HH_OK ? d.op : 0;
        B.status[b] = st;
    }
}

template <uint32_t R, uint32_t S>
hipError_t launch_ring(const Lz4Batch &B, hipStream_t s) {
    constexpr uint32_t lds = ring::RingDec<R, S>::kLds;
    hipError_t e = hipFuncSetAttribute((const void *)lz4_ring_kernel<R, S>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((lz4_ring_kernel<R, S>), dim3(B.nblocks), dim3(64), lds, s, B);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_lz4_ring(const Lz4Batch &B, uint32_t ring_kib, hipStream_t s) {
    if (B.nblocks == 0) return hipSuccess;
    switch (ring_kib) {
        case 8: return launch_ring<8192, 2048>(B, s);
        case 16: return launch_ring<16384, 3072>(B, s);
        case 32: return launch_ring<32768, 4096>(B, s);
        default: return launch_ring<4096, 4096>(B, s);
    }
}

}  // namespace hh
