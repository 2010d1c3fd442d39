// pkv_probe.hip — HBM calibration probes for the roofline of the decode engine.
//
// The MI355X counterpart of the reference's micro_benchmarks/01_hbm_bandwidth.cu:20-51
// (hbm_read / hbm_copy kernels): streaming kernels of known size, used to
//   * measure the achievable read bandwidth of this GPU for the decode kernel's own
//     access patterns (roofline denominator next to the 8 TB/s peak), and
//   * calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE against a known byte count.
// Patterns over 4 KB chunks (one 16-token page slab of one KV head):
//   0  contiguous: each 16-byte load instruction covers 1 KB of consecutive bytes
//   1  K operand:  each instruction reads 16 rows x 64 B (the decode kernel's K loads)
//   2  V operand:  each instruction reads 4 rows x 256 B (the decode kernel's V loads)
//   3  K through LDS: the loads of pattern 2 (whole 128-byte lines), then each chunk is
//      written to a per-wave LDS slab and read back in the K-operand layout (16 rows x
//      64 B per read), with the 16-byte column index XORed with the row so that neither
//      the writes nor the reads conflict on LDS banks (pkv_probe_read_inflight only)
// Chunks are visited in a pseudo-random order (as random page ids would be).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv.h"  // status codes
#include "pkv_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kRsrcWord3 = 0x00020000u;

__device__ inline uint32_t lane_offset(int pattern, int lane, int k) {
  const int c = lane & 15, g = lane >> 4;
  if (pattern == 1) return c * 256 + k * 64 + g * 16;       // K operand (k = 0..3)
  if (pattern >= 2) return (4 * g + k) * 256 + c * 16;      // V operand / whole lines
  return k * 1024 + lane * 16;                              // contiguous
}

// Swizzled LDS byte offset of 16-byte column `col` of row `row` in a 16 x 256 B slab.
__device__ inline uint32_t slab_offset(int row, int col) {
  return row * 256 + ((col ^ (row & 7)) * 16);
}

// Pattern 3: a chunk loaded as whole lines (lane (c, g) holds rows 4g + k, column c) goes
// through the wave's LDS slab and comes back as K operands (row c, columns 4k + g).
__device__ inline void through_lds(u32x4 (&v)[4], uint8_t* slab, int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) *(u32x4*)(slab + slab_offset(4 * g + k, c)) = v[k];
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = *(const u32x4*)(slab + slab_offset(c, 4 * k + g));
  __builtin_amdgcn_wave_barrier();
}

// One wave reads whole 4 KB chunks (4 loads of 1 KB); 4 chunks in flight per iteration.
__global__ __launch_bounds__(512) void probe_read_kernel(const uint8_t* src, uint64_t chunks,
                                                         uint64_t stride, int pattern,
                                                         uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int waves_per_group = blockDim.x >> 6;
  const uint64_t wave = (uint64_t)blockIdx.x * waves_per_group + (threadIdx.x >> 6);
  const uint64_t nwaves = (uint64_t)gridDim.x * waves_per_group;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint64_t base = wave; base < chunks; base += 4 * nwaves) {
    u32x4 v[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint64_t idx = base + u * nwaves;
      const uint64_t chunk = (idx * stride) % chunks;  // stride coprime to chunks: permutation
      const int nrec = idx < chunks ? 4096 : 0;
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(src + chunk * 4096), (short)0, __builtin_amdgcn_readfirstlane(nrec), kRsrcWord3);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[u][k] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_offset(pattern, lane, k), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc ^= v[u][k];
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[blockIdx.x] = x;  // keeps the loads alive; practically never true
}

// Per-CU bandwidth against bytes in flight: each wave keeps U chunks (U x 4 KB) in flight
// and workgroups have `blockDim.x / 64` waves (4, 8 or 16).
template <int U>
__global__ __launch_bounds__(1024) void probe_inflight_kernel(const uint8_t* src, uint64_t chunks,
                                                              uint64_t stride, int pattern,
                                                              uint32_t* sink) {
  extern __shared__ uint8_t lds[];  // 96 KB: one workgroup per CU; 4 KB slab per wave
  uint8_t* slab = lds + (threadIdx.x >> 6) * 4096;
  const int lane = threadIdx.x & 63;
  const int waves_per_group = blockDim.x >> 6;
  const uint64_t wave = (uint64_t)blockIdx.x * waves_per_group + (threadIdx.x >> 6);
  const uint64_t nwaves = (uint64_t)gridDim.x * waves_per_group;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint64_t base = wave; base < chunks; base += U * nwaves) {
    u32x4 v[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t idx = base + u * nwaves;
      const uint64_t chunk = (idx * stride) % chunks;
      const int nrec = idx < chunks ? 4096 : 0;
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(src + chunk * 4096), (short)0, __builtin_amdgcn_readfirstlane(nrec), kRsrcWord3);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[u][k] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_offset(pattern, lane, k), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (pattern == 3) through_lds(v[u], slab, lane);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc ^= v[u][k];
    }
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[blockIdx.x] = x;
}

__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4* src, u32x4* dst, uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 4096) of `src` once with access pattern `pattern`
// (0 contiguous, 1 K operand, 2 V operand) over 4 KB chunks in a permuted order.
int pkv_probe_read(const void* src, size_t bytes, int32_t pattern, void* sink, void* stream) {
  if (!src || !sink || bytes < 4096 || bytes % 4096 || bytes / 4096 >= 2147483647ull ||
      pattern < 0 || pattern > 2)
    return PKV_ERR_INVALID_ARGUMENT;
  const uint64_t chunks = bytes / 4096;
  // 2^31 - 1 is prime, so its residue is coprime to any smaller chunk count: the visit
  // order idx * stride mod chunks is a permutation.
  const uint64_t stride = chunks > 1 ? 2147483647ull % chunks : 1;
  hipLaunchKernelGGL(probe_read_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, chunks, stride ? stride : 1, pattern, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? PKV_OK : PKV_ERR_LAUNCH;
}

// pkv_probe_read with `workgroups` workgroups of 8 waves, each holding 96 KB of LDS so
// that no two share a CU: with fewer workgroups than CUs it measures what a given number
// of CUs can stream (sink must hold `workgroups` words).
int pkv_probe_read_cus(const void* src, size_t bytes, int32_t pattern, int32_t workgroups,
                       void* sink, void* stream) {
  if (!src || !sink || bytes < 4096 || bytes % 4096 || bytes / 4096 >= 2147483647ull ||
      pattern < 0 || pattern > 2 || workgroups <= 0 || workgroups > 65536)
    return PKV_ERR_INVALID_ARGUMENT;
  const uint64_t chunks = bytes / 4096;
  const uint64_t stride = chunks > 1 ? 2147483647ull % chunks : 1;
  hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(512), 96 * 1024, (hipStream_t)stream,
                     (const uint8_t*)src, chunks, stride ? stride : 1, pattern, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? PKV_OK : PKV_ERR_LAUNCH;
}

// pkv_probe_read_cus with `waves` (4, 8 or 16) waves per workgroup, each keeping
// `chunks_per_wave` (1, 2 or 4) chunks of 4 KB in flight; pattern 3 also moves every
// chunk through LDS (at most 16 waves x 4 KB of the workgroup's 96 KB).
int pkv_probe_read_inflight(const void* src, size_t bytes, int32_t pattern, int32_t waves,
                            int32_t chunks_per_wave, int32_t workgroups, void* sink, void* stream) {
  if (!src || !sink || bytes < 4096 || bytes % 4096 || bytes / 4096 >= 2147483647ull ||
      pattern < 0 || pattern > 3 || workgroups <= 0 || workgroups > 65536 ||
      (waves != 4 && waves != 8 && waves != 16) ||
      (chunks_per_wave != 1 && chunks_per_wave != 2 && chunks_per_wave != 4))
    return PKV_ERR_INVALID_ARGUMENT;
  const uint64_t chunks = bytes / 4096;
  const uint64_t stride = chunks > 1 ? 2147483647ull % chunks : 1;
  const dim3 grid(workgroups), block(waves * 64);
  const size_t lds = 96 * 1024;  // at most one workgroup per CU
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* p = (const uint8_t*)src;
  const uint64_t st = stride ? stride : 1;
  if (chunks_per_wave == 1)
    hipLaunchKernelGGL(probe_inflight_kernel<1>, grid, block, lds, s, p, chunks, st, pattern, (uint32_t*)sink);
  else if (chunks_per_wave == 2)
    hipLaunchKernelGGL(probe_inflight_kernel<2>, grid, block, lds, s, p, chunks, st, pattern, (uint32_t*)sink);
  else
    hipLaunchKernelGGL(probe_inflight_kernel<4>, grid, block, lds, s, p, chunks, st, pattern, (uint32_t*)sink);
  return hipGetLastError() == hipSuccess ? PKV_OK : PKV_ERR_LAUNCH;
}

// Copies `bytes` (a multiple of 16) from src to dst with a plain grid-stride kernel.
int pkv_probe_copy(const void* src, void* dst, size_t bytes, void* stream) {
  if (!src || !dst || bytes == 0 || bytes % 16) return PKV_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(probe_copy_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)src, (u32x4*)dst, (uint64_t)(bytes / 16));
  return hipGetLastError() == hipSuccess ? PKV_OK : PKV_ERR_LAUNCH;
}

}  // extern "C"
