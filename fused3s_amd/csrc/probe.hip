// probe.hip -- measurement only: the random-gather ceiling of the device for
// the access pattern of the fused pass (no reference counterpart).
//
// Each wave takes `cpw` steps of 32 columns; per column it loads the 128-byte
// row (one head) of K and of V, eight lanes per row with one 16-byte buffer
// load each -- four load instructions per 32 rows, the fused pass's own load
// shape -- and folds what it loaded into one word per wave, so no load is
// dead code.  The rate it reaches over uniformly random rows is what the
// vector-memory path and the memory below the L2 sustain for 128-byte
// gathers; the fused pass does more work per row and is priced against it.
#include "f3s_common.hpp"
#include "f3s_device.hpp"

namespace f3s {

namespace {

typedef uint32_t pu4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256)
gather_probe_kernel(const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                    uint32_t table_bytes, uint32_t row_stride, const int32_t* __restrict__ idx,
                    int64_t nsteps, int32_t cpw, uint32_t* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t s0 = wave * cpw;
    if (s0 >= nsteps) return;
    const int64_t s1 = s0 + cpw < nsteps ? s0 + cpw : nsteps;
    // offsets at or past table_bytes read 0 (the descriptor's range check)
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(K), (short)0, (int)table_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(V), (short)0, (int)table_bytes, 0x00020000);
    const uint32_t piece = 16u * (lane & 7);
    pu4 acc = {0u, 0u, 0u, 0u};
    for (int64_t s = s0; s < s1; ++s) {
        const int32_t my = idx[s * 32 + (lane & 31)];
        pu4 kk[4], vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 64-bit offset, clamped to table_bytes: a negative row or one
            // past the table reads zero through the descriptor's range check
            const int64_t row = __shfl(my, (lane >> 3) + 8 * i);
            const int64_t o = row * (int64_t)row_stride + piece;
            const uint32_t off = (o >= 0 && o < (int64_t)table_bytes) ? (uint32_t)o : table_bytes;
            kk[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
            vv[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc ^= kk[i] ^ vv[i];
    }
    uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o);
    if (lane == 0) out[wave] = x;
}

}  // namespace

}  // namespace f3s

using namespace f3s;

extern "C" f3s_status f3s_probe_gather(const uint16_t* K, const uint16_t* V, int64_t rows,
                                       int32_t row_stride, const int32_t* d_idx, int64_t count,
                                       int32_t cpw, uint32_t* d_out, void* stream)
{
    F3S_REQUIRE(K && V && d_idx && d_out, "f3s_probe_gather: NULL pointer");
    F3S_REQUIRE(rows > 0 && row_stride >= 128 && row_stride % 16 == 0,
                "f3s_probe_gather: bad table shape");
    F3S_REQUIRE(rows * (int64_t)row_stride <= (int64_t)0xffff0000u,
                "f3s_probe_gather: table past 32-bit buffer offsets");
    F3S_REQUIRE(count > 0 && count % 32 == 0, "f3s_probe_gather: count must be a multiple of 32");
    F3S_REQUIRE(cpw >= 1 && cpw <= 1024, "f3s_probe_gather: cpw out of range");
    F3S_TRY(require_device());
    clear_error();
    const int64_t nsteps = count / 32;
    const int64_t waves = (nsteps + cpw - 1) / cpw;
    const int64_t blocks = (waves + 3) / 4;
    F3S_REQUIRE(blocks < ((int64_t)1 << 31), "f3s_probe_gather: too many steps");
    hipLaunchKernelGGL(gather_probe_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       as_stream(stream), K, V, (uint32_t)(rows * row_stride),
                       (uint32_t)row_stride, d_idx, nsteps, cpw, d_out);
    F3S_HIP(hipGetLastError());
    return F3S_OK;
}
