// pkv_append.hip — writes each row's newest token (K and V) into its tail page: the
// producer side of the paged pool the decode kernels read.
//
// The reference never writes K/V: its harness only grows the lengths
// (tests/benchmark_serving_trace.py:285-298), and the paper lists fused KV-cache writes as
// future work (paper/persistentkv_mlsys_workshop.tex:689).  A serving loop writes the new
// token before its decode step; this is that write on the GPU.  The fp8 variant quantises
// to OCP e4m3 with a per-tensor scale, the inverse of the fp8 decode ops' dequantisation.
//
// Row b's token goes to position seq_lens[b] - 1: page block_table[b, pos / ps], slot
// pos % ps of the [pages, Hkv, ps, 128] pools.  Rows with no tokens, or whose position or
// page falls outside the table or the pool, are skipped, so no write leaves the pools.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "pkv.h"
#include "pkv_e4m3.h"

namespace pkv {
int fail(int status, const char* fmt, ...);  // pkv_decode.hip: sets pkv_last_error()
int ok();
}  // namespace pkv

namespace {

constexpr int kD = 128;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)

// A pointer that is the same in every lane of the wave, as buffer descriptors need.
__device__ inline void* wave_ptr(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return (void*)(((uint64_t)hi << 32) | lo);
}

struct AppendArgs {
  const uint8_t* k_new;   // [B, Hkv, 128], 2-byte elements
  const uint8_t* v_new;
  uint8_t* k_pages;       // [num_pages, Hkv, ps, 128], 2- or 1-byte elements
  uint8_t* v_pages;
  const int32_t* block_table;  // [B, max_pages]
  const int32_t* seq_lens;     // [B], lengths after the append
  int32_t batch, hkv, page_size, max_pages, num_pages;
  float k_scale, v_scale;      // fp8 pools: stored value = e4m3(x / scale)
};

// One wave per (row, kv head); lane l writes dims 2l and 2l + 1 of K and of V.
template <bool FP8, bool BF16_IN>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  const int wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave_id >= a.batch * a.hkv) return;
  const int row = wave_id / a.hkv, h = wave_id - row * a.hkv;
  // Straight-line code with no early return, so that the new token's loads stay ahead of
  // (and overlap) the dependent seq_lens -> block_table reads that place it.  A skipped
  // row stores through a descriptor of 0 bytes, which the hardware drops.
  const long src = ((long)row * a.hkv + h) * kD + 2 * lane;  // element index
  const uint32_t k2 = *(const uint32_t*)(a.k_new + src * 2);
  const uint32_t v2 = *(const uint32_t*)(a.v_new + src * 2);
  const int pos = a.seq_lens[row] - 1;
  const int logical = pos < 0 ? 0 : pos / a.page_size;
  const bool in_table = pos >= 0 && logical < a.max_pages;
  const int page = a.block_table[(long)row * a.max_pages + (in_table ? logical : 0)];
  const bool valid = in_table && page >= 0 && page < a.num_pages;
  constexpr int kElem = FP8 ? 1 : 2;
  const long slot = valid ? (((long)page * a.hkv + h) * a.page_size + pos % a.page_size) * kD : 0;
  const int nrec = __builtin_amdgcn_readfirstlane(valid ? kD * kElem : 0);
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(wave_ptr(a.k_pages + slot * kElem), (short)0, nrec, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(wave_ptr(a.v_pages + slot * kElem), (short)0, nrec, kRsrcWord3);
  if constexpr (FP8) {
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)pkv::e4m3_pack2<BF16_IN>(k2, a.k_scale), rk,
                                          lane * 2, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)pkv::e4m3_pack2<BF16_IN>(v2, a.v_scale), rv,
                                          lane * 2, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(k2, rk, lane * 4, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(v2, rv, lane * 4, 0, 0);
  }
}

int run_append(const void* k_new, const void* v_new, void* k_pages, void* v_pages,
               const int32_t* block_table, const int32_t* seq_lens, int32_t batch,
               int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
               int32_t max_pages, bool fp8, float k_scale, float v_scale, int32_t dtype,
               void* stream) {
  using pkv::fail;
  if (batch < 0 || num_kv_heads <= 0 || page_size <= 0 || max_pages <= 0 || num_pages <= 0)
    return fail(PKV_ERR_INVALID_ARGUMENT,
                "append: batch %d, num_kv_heads %d, page_size %d, max_pages %d, num_pages %d",
                batch, num_kv_heads, page_size, max_pages, num_pages);
  if (head_dim != kD) return fail(PKV_ERR_UNSUPPORTED, "append: head_dim %d (only 128)", head_dim);
  if (dtype != PKV_DTYPE_F16 && dtype != PKV_DTYPE_BF16)
    return fail(PKV_ERR_INVALID_ARGUMENT, "append: unknown dtype %d", dtype);
  if (fp8 && !(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY))
    return fail(PKV_ERR_INVALID_ARGUMENT, "append: k_scale and v_scale must be finite and positive");
  if ((long)batch * num_kv_heads > (1L << 30))
    return fail(PKV_ERR_INVALID_ARGUMENT, "append: batch * num_kv_heads too large");
  if (batch == 0) return pkv::ok();
  if (!k_new || !v_new || !k_pages || !v_pages || !block_table || !seq_lens)
    return fail(PKV_ERR_INVALID_ARGUMENT, "append: null pointer");
  const AppendArgs a{(const uint8_t*)k_new, (const uint8_t*)v_new, (uint8_t*)k_pages,
                     (uint8_t*)v_pages, block_table, seq_lens, batch, num_kv_heads,
                     page_size, max_pages, num_pages, k_scale, v_scale};
  const dim3 grid((unsigned)((batch * num_kv_heads + 3) / 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  const bool bf16 = dtype == PKV_DTYPE_BF16;
  if (!fp8) append_kernel<false, false><<<grid, block, 0, s>>>(a);  // a 4-byte copy per lane
  else if (bf16) append_kernel<true, true><<<grid, block, 0, s>>>(a);
  else append_kernel<true, false><<<grid, block, 0, s>>>(a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? pkv::ok() : fail(PKV_ERR_LAUNCH, "append launch: %s", hipGetErrorString(e));
}

}  // namespace

extern "C" {

int pkv_append_kv(const void* k_new, const void* v_new, void* k_pages, void* v_pages,
                  const int32_t* block_table, const int32_t* seq_lens, int32_t batch,
                  int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
                  int32_t max_pages, int32_t dtype, void* stream) {
  return run_append(k_new, v_new, k_pages, v_pages, block_table, seq_lens, batch, num_kv_heads,
                    head_dim, num_pages, page_size, max_pages, false, 1.f, 1.f, dtype, stream);
}

int pkv_append_kv_fp8(const void* k_new, const void* v_new, void* k_pages, void* v_pages,
                      const int32_t* block_table, const int32_t* seq_lens, int32_t batch,
                      int32_t num_kv_heads, int32_t head_dim, int32_t num_pages,
                      int32_t page_size, int32_t max_pages, float k_scale, float v_scale,
                      int32_t dtype, void* stream) {
  return run_append(k_new, v_new, k_pages, v_pages, block_table, seq_lens, batch, num_kv_heads,
                    head_dim, num_pages, page_size, max_pages, true, k_scale, v_scale, dtype,
                    stream);
}

}  // extern "C"
