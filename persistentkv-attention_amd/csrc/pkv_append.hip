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
  const int pos = a.seq_lens[row] - 1;
  if (pos < 0) return;
  const int logical = pos / a.page_size;
  if (logical >= a.max_pages) return;
  const int page = a.block_table[(long)row * a.max_pages + logical];
  if (page < 0 || page >= a.num_pages) return;
  const long src = ((long)row * a.hkv + h) * kD + 2 * lane;  // element index
  const long dst = (((long)page * a.hkv + h) * a.page_size + pos % a.page_size) * kD + 2 * lane;
  const uint32_t k2 = *(const uint32_t*)(a.k_new + src * 2);
  const uint32_t v2 = *(const uint32_t*)(a.v_new + src * 2);
  if constexpr (FP8) {
    *(uint16_t*)(a.k_pages + dst) = (uint16_t)pkv::e4m3_pack2<BF16_IN>(k2, a.k_scale);
    *(uint16_t*)(a.v_pages + dst) = (uint16_t)pkv::e4m3_pack2<BF16_IN>(v2, a.v_scale);
  } else {
    *(uint32_t*)(a.k_pages + dst * 2) = k2;
    *(uint32_t*)(a.v_pages + dst * 2) = v2;
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
