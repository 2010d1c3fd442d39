// pkv_decode.hip — paged GQA decode attention for MI355X (gfx950, CDNA4).
//
// One workgroup (8 wave64s when G <= 16, 4 when G > 16) owns one unit of work: a
// (row, kv head) pair and a range of 32-token tiles.  The unit is a whole row (direct
// op), one sequence split of a row (grid-split ops) or one compact work item (work-queue
// op).  The waves stream disjoint sub-ranges of the unit's tiles, so one K/V fetch from
// HBM serves all G query heads of the KV group, then combine their online-softmax states
// through LDS.  K/V come from paged pools (fp16 / bf16, or fp8 e4m3 unpacked exactly in
// registers) or from the contiguous [B, Hkv, N, 128] layout.
//
// Per wave and 32-token tile:
//   * K and V rows are read straight into VGPRs in MFMA operand layout with 16-byte
//     buffer loads (8-byte for fp8).  Each 16-token block of a page gets its own buffer
//     descriptor whose size covers only the block's valid rows, so rows at or past seq_len
//     read as zero and no access can leave the page.
//   * S^T[token, head] = K * Q^T with v_mfma_f32_16x16x32 (heads padded to 16 per block).
//   * Online softmax in base 2 (v_exp_f32); the running max is wave-uniform per head.
//   * O[head, dim] += P * V with the same MFMA; V is transposed in registers by byte
//     permutes so that each lane holds 8 tokens of one dim (the MFMA k operand).
// Partial states keep the reference's workspace format: m in natural-log units of the
// scaled score, l = sum exp(s - m), acc = sum exp(s - m) v.
//
// Reference: kernels/persistentkv_attention.cuh (decode kernel :270-717, merges
// :719-784, launches :929-1261), tests/persistentkv_torch_extension.cu (op checks).

#include <hip/hip_runtime.h>

#include <float.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

#include "pkv.h"

namespace pkv {

constexpr int kD = 128;              // head dim (cuh:26)
constexpr int kTile = 32;            // work-item tile in tokens (cuh:28)
constexpr int kMaxWaves = 8;         // waves per workgroup: 4 or 8 (template NW)
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)
// Cache policy of the K/V page loads: non-temporal (the buffer instructions' nt bit).
// Every K/V byte is read once per launch, so keeping it out of the caches leaves L2 to
// the metadata that dependent load chains wait on (block tables, work items, query rows).
// Measured against the default policy: C4 decode 45.8 -> 43.3 us, C3 32k op 31.0 -> 28.2
// us, C2 op 118.6 -> 109.0 us.
constexpr int kKvLoadPolicy = 2;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// softmax scale 1/sqrt(128) (cuh:944) folded with log2(e) for exp2-based softmax.
constexpr float kScaleLog2 = 0.08838834764831845f * 1.4426950408889634f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

enum Mode : int { kDirect = 0, kSplit = 1, kQueue = 2 };

// ---------------------------------------------------------------------------------
// Element types.  P (softmax weights) enters the PV product in the KV dtype; bf16 keeps
// 8 mantissa bits, so its P is split into hi + lo terms (two MFMAs) to stay well inside
// the 2e-3 tolerance.
// ---------------------------------------------------------------------------------
struct Half {
  static constexpr int kPasses = 1;
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Two floats to 2 x fp16 (round to nearest even), a in the low half.
  __device__ static inline uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  // fp8 (OCP e4m3) bytes 2*HI and 2*HI + 1 of x to 2 x fp16 (exact).
  template <bool HI>
  __device__ static inline uint32_t fp8_pair(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)x, 1.0f, HI));
  }
  // 8 fp8 (OCP e4m3) values, byte i of the pair = element i, to 8 fp16 (exact).
  __device__ static inline u32x4 unpack8(u32x2 x) {
    return u32x4{fp8_pair<false>(x[0]), fp8_pair<true>(x[0]), fp8_pair<false>(x[1]), fp8_pair<true>(x[1])};
  }
};

struct BFloat {
  static constexpr int kPasses = 2;
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Two floats to 2 x bf16 (round to nearest even), a in the low half.
  __device__ static inline uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  // fp8 (OCP e4m3) bytes 2*HI and 2*HI + 1 of x to 2 x bf16 (exact).
  template <bool HI>
  __device__ static inline uint32_t fp8_pair(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)x, 1.0f, HI));
  }
  // 8 fp8 (OCP e4m3) values to 8 bf16 (exact).
  __device__ static inline u32x4 unpack8(u32x2 x) {
    return u32x4{fp8_pair<false>(x[0]), fp8_pair<true>(x[0]), fp8_pair<false>(x[1]), fp8_pair<true>(x[1])};
  }
};

struct DecodeArgs {
  const uint8_t* q;           // [q_rows, Hq, 128]
  const uint8_t* k_pages;     // [num_pages, Hkv, ps, 128]
  const uint8_t* v_pages;
  const int32_t* block_table; // [B, max_pages]
  const int32_t* seq_lens;    // [B] or null: every row has `context` tokens
  const int32_t* q_indices;   // [B] or null
  const int32_t* out_indices; // [B] or null
  const int32_t* work_items;  // [num_tasks, 5] (queue mode)
  const int32_t* split_offsets;  // [B + 1] (queue mode)
  int32_t* merge_counters;    // [B, Hkv] or null (queue mode, fused merge)
  uint8_t* out;               // [out_rows, Hq, 128] (direct mode, fused merge)
  float* part_m;              // workspace partition (split / queue modes)
  float* part_l;
  float* part_acc;
  int32_t batch, hq, hkv, group;
  int32_t q_rows, out_rows;
  int32_t context;            // tokens per row when seq_lens is null
  int32_t page_size, page_shift;  // page_shift = log2(page_size) or -1
  int32_t max_pages, num_pages;
  int32_t num_splits;         // split mode
  int32_t num_tasks, total_slots;  // queue mode
  // Scores are q.k * score_scale in log2 units (1/sqrt(128) * log2(e), times the K
  // dequantisation scale for fp8 K); outputs and partial accumulators are scaled by
  // v_scale (the V dequantisation scale; 1 otherwise).
  float score_scale, v_scale;
  int32_t kv_fp8;             // K/V are fp8 (OCP e4m3) with 1-byte elements
  // Contiguous layout only: unit kv head v reads the K/V of head v / kv_div (1, or G for
  // the query-head baseline, whose units are single query heads).
  int32_t kv_div;
  // Fused append (paged fp16 / bf16, pages a multiple of 16), else null: each row's
  // newest token, [B, Hkv, 128] in the KV dtype, written to position seq_lens[b] - 1.
  const uint8_t* k_new;
  const uint8_t* v_new;
  // Balanced schedule only: per (row, kv head) pair, {first wave, waves, T low, T high} of
  // its tiles, written by the decode for the merge (16-byte entries, 16-byte aligned), and
  // per decode workgroup the result of its part of the queue check (1 = passed).
  int32_t* bal_plan;
  int32_t* bal_flags;
};

// ---------------------------------------------------------------------------------
// Small device helpers.
// ---------------------------------------------------------------------------------
__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ inline void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return (void*)(((uint64_t)hi << 32) | lo);
}

// A row length as the kernels use it.  The reference trusts seq_lens (cuh:217-219);
// clamping to the table width keeps every page lookup inside the row for any input.
__device__ inline int clamp_length(const DecodeArgs& a, int len) {
  const long cap = (long)a.max_pages * a.page_size;
  if (len > cap) len = (int)cap;
  return len < 0 ? 0 : len;
}
__device__ inline int row_length(const DecodeArgs& a, int row) {
  return clamp_length(a, a.seq_lens ? a.seq_lens[row] : a.context);
}

__device__ inline int clamp_page(const DecodeArgs& a, int page) {
  // Out-of-range table entries are clamped into the pool (the reference reads
  // whatever the entry addresses); valid tables are unaffected.
  return (unsigned)page < (unsigned)a.num_pages ? page : (page < 0 ? 0 : a.num_pages - 1);
}

__device__ inline void page_of(const DecodeArgs& a, int token, int& logical, int& offset) {
  if (a.page_shift >= 0) {
    logical = token >> a.page_shift;
    offset = token & (a.page_size - 1);
  } else {
    logical = token / a.page_size;
    offset = token - logical * a.page_size;
  }
}

// Token held by V-operand slot j (0..7) of lane group g within a 32-token tile.  It
// matches the token order of the score fragments: slots 0-3 are S^T rows 4g..4g+3 of
// the first 16-token block, slots 4-7 the same rows of the second block.
__device__ inline int v_slot_token(int g, int j) { return (j >> 2) * 16 + 4 * g + (j & 3); }

// ---------------------------------------------------------------------------------
// Cross-lane helpers.  Lanes l, l^16, l^32, l^48 hold the same head in the score
// layout.  These run on the first tile, on the rare rescale and once per range, so the
// LDS-routed shuffles are off the hot path.  (v_permlane{16,32}_swap would avoid LDS, but
// the compiler folds max/sum of the two results of a swap with identical operands into a
// single operand, which drops the exchange.)
// ---------------------------------------------------------------------------------
__device__ inline float head_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float head_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Scalar (SMEM) load of a wave-uniform int: block-table entries are read through the
// constant address space so that waiting for them never waits for K/V vector loads.
__device__ inline int load_scalar(const int32_t* p) {
  return uniform(*(const __attribute__((address_space(4))) int32_t*)p);
}

// Vector (buffer) load of a wave-uniform int.  Unlike a scalar load, whose completion can
// only be waited for together with every other scalar load in flight (kernel-argument
// reads included), it completes in issue order with the wave's other vector loads.
__device__ inline int load_vector_uniform(const int32_t* p) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(p), (short)0, 4, kRsrcWord3);
  return uniform((int)__builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0));
}
// The same load issued without waiting for it: the result stays in a VGPR (0 when p is
// null, which reads nothing) until uniform() is applied where it is used.
__device__ inline int load_vector_deferred(const int32_t* p) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(p), (short)0, p ? 4 : 0, kRsrcWord3);
  return (int)__builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
}
// load_vector_deferred whose result the compiler must treat as per-lane, so it is not
// copied to an SGPR (and waited for) at once: its offset is `lane_zero`, a per-lane value
// that is 0 at run time but not provably so.
__device__ inline int load_vector_lanes(const int32_t* p, int lane_zero) {
  const int zero = lane_zero;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(p), (short)0, p ? 4 : 0, kRsrcWord3);
  return (int)__builtin_amdgcn_raw_buffer_load_b32(r, zero, 0, 0);
}

// ---------------------------------------------------------------------------------
// Page loaders.  A wave streams tiles [t0, t1) of one (row, kv head); tokens at or past
// `lim` = min(row length, 32 * t1) are never read.  Each loader splits a tile into
// lookup() (block-table reads, issued two tiles ahead) and issue() (the 16 K/V loads).
//
// FastPager: page sizes that are multiples of 16, so each 16-token block lies inside one
// page.  The page id is wave-uniform (scalar load) and each block gets a buffer
// descriptor covering only its valid rows: rows past `lim` read as zero without a
// memory request, and no access can leave the block.
// GenericPager: any other page size, per-lane table lookups and predicated loads.
// ---------------------------------------------------------------------------------
struct TileRegs {
  u32x4 k[2][4];  // k[b][kk]: K row (block b, token c), dims 32kk + 8g .. +8
  u32x4 v[8];     // v[j]: V row of token slot j (v_slot_token), dims 8c .. +8
};

// fp8 K/V tile as loaded.  K: lane (g, c) holds 16 bytes of token c (+ 16b) per half h,
// dims 64h + 16g .. +16; MFMA k-block kk takes the 8 bytes at dims 64(kk/2) + 16g +
// 8(kk%2), and Q is loaded with the same dims (load_q<HB, true>).  A 16-byte load per lane
// takes half of each 128-byte token row per instruction, as the 2-byte K loads do; 8-byte
// loads (a quarter row, four requests per line) held the fp8 decode to 0.47 of 8 TB/s
// against 0.61 with this layout.  V: the same lanes and rows as TileRegs, 8 one-byte
// elements per 16-byte fp16 chunk.
struct Fp8Tile {
  u32x4 k[2][2];
  u32x2 v[8];
};

// Each pager's issue() fills a Raw tile, which compute_tile reads through tile_k / transpose_v
// (fp8 tiles are unpacked there).
struct FastPager {
  struct Pages {
    int page[2];  // physical page of each 16-token block (unused when the block is empty)
  };
  using Raw = TileRegs;
  const DecodeArgs& a;
  const int32_t* trow;
  int lim;
  long head_bytes;   // kvh * ps * 256
  long page_bytes;   // Hkv * ps * 256
  uint32_t koff[4];  // per-lane byte offsets inside a block, K (per 32-dim step)
  uint32_t voff[8];  // per-lane byte offsets inside a block, V (per token slot)

  __device__ FastPager(const DecodeArgs& args, int row, int kvh, int limit, int lane)
      : a(args), lim(limit) {
    trow = a.block_table + (long)row * a.max_pages;
    head_bytes = (long)kvh * a.page_size * (kD * 2);
    page_bytes = (long)a.hkv * a.page_size * (kD * 2);
    const int c = lane & 15, g = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) koff[kk] = c * 256 + kk * 64 + g * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) voff[j] = (4 * g + (j & 3)) * 256 + c * 16;
  }

  // Table reads do not depend on the row length (columns are clamped to the table), so
  // the first ones can be issued as soon as the work item is known.
  __device__ inline Pages lookup(int tile) const {
    Pages p;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int tok0 = (tile < 0 ? 0 : tile) * kTile + b * 16;
      int logical, in_page;
      page_of(a, tok0, logical, in_page);
      logical = logical < a.max_pages ? logical : a.max_pages - 1;
      p.page[b] = load_scalar(trow + logical);  // clamped in issue(), after the compute
    }
    return p;
  }

  // K and V buffer descriptors of 16-token block b of `tile`, covering only its valid rows.
  __device__ inline void block_rsrc(int tile, int b, const Pages& p, __amdgpu_buffer_rsrc_t& rk,
                                    __amdgpu_buffer_rsrc_t& rv) const {
    const int tok0 = tile * kTile + b * 16;
    int nvalid = lim - tok0;
    nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
    int logical, in_page;
    page_of(a, tok0, logical, in_page);
    const long off = nvalid > 0
        ? (long)clamp_page(a, p.page[b]) * page_bytes + head_bytes + (long)in_page * (kD * 2) : 0;
    // Descriptors must be wave-uniform (SGPRs); readfirstlane states that to the
    // compiler, which otherwise wraps every buffer load in a waterfall loop.
    const int nrec = uniform(nvalid * (kD * 2));
    rk = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.k_pages + off), (short)0, nrec, kRsrcWord3);
    rv = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.v_pages + off), (short)0, nrec, kRsrcWord3);
  }

  __device__ inline void issue(int tile, const Pages& p, TileRegs& r) const {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      __amdgpu_buffer_rsrc_t rk, rv;
      block_rsrc(tile, b, p, rk, rv);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) r.k[b][kk] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff[kk], 0, kKvLoadPolicy);
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[b * 4 + j] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff[b * 4 + j], 0, kKvLoadPolicy);
    }
  }
};

// FastPager for a step that also appends each row's newest token, the write of
// pkv_append_kv: position seq_lens[row] - 1, page block_table[row, pos / ps].  That
// token's K and V rows are taken from k_new / v_new instead of the pool, and the wave
// whose tiles hold it also writes it into the pool.  No other wave of the launch reads
// those bytes (each row's tail slot belongs to one (row, kv head) unit), so the result
// equals pkv_append_kv followed by the same decode.  Rows whose append pkv_append_kv
// skips (no tokens, a position past the table, a page id outside the pool) are decoded
// from the pool as they are.
struct AppendPager : FastPager {
  int pos;             // the new token's position, or -1 when this wave does not hold it
  int lane;
  const uint8_t* kn;   // k_new[row, kvh, :], 256 bytes
  const uint8_t* vn;

  __device__ AppendPager(const DecodeArgs& args, int row, int kvh, int limit, int lane_id)
      : FastPager(args, row, kvh, limit, lane_id), lane(lane_id) {
    const int raw = load_scalar(args.seq_lens + row);
    const long cap = (long)args.max_pages * args.page_size;
    // limit = min(32 * t1, clamped length): the token is this wave's when its tile is
    // below t1 (tiles below t0 are never issued).
    pos = raw >= 1 && (long)raw <= cap && raw - 1 < limit ? raw - 1 : -1;
    const long src = ((long)row * args.hkv + kvh) * (kD * 2);
    kn = args.k_new + src;
    vn = args.v_new + src;
  }

  // The new token's row in `tile` (0 .. 31), or -1 when the tile does not hold it or the
  // append skips the row (its page id is outside the pool).  Wave-uniform.
  __device__ inline int new_row(int tile, const Pages& p) const {
    const int rel = pos - tile * kTile;
    if (pos < 0 || rel < 0 || rel >= kTile) return -1;
    const int page = (rel >> 4) ? p.page[1] : p.page[0];
    return (unsigned)page < (unsigned)a.num_pages ? rel : -1;
  }

  // Takes the new token's V row (and, with K_REGS, its K row) from v_new / k_new into the
  // tile's registers and writes both rows into the pools.  Lane (c, g) holds K row c of
  // each block at bytes 64kk + 16g, and V row 4g + jj of block slot jj at bytes 16c
  // (FastPager's koff / voff).  The lanes that hold the token reload those registers; the
  // loads return in issue order, after the pool loads of the same registers.
  template <bool K_REGS>
  __device__ inline void take_new(int rel, const Pages& p, TileRegs& r) const {
    const int b = rel >> 4, prow = rel & 15;
    const int c = lane & 15, g = lane >> 4;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      if (K_REGS && bb == b && c == prow) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) r.k[bb][kk] = *(const u32x4*)(kn + kk * 64 + g * 16);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        if (bb == b && 4 * g + jj == prow) r.v[bb * 4 + jj] = *(const u32x4*)(vn + c * 16);
    }
    const int page = b ? p.page[1] : p.page[0];
    int logical, in_page;
    page_of(a, pos, logical, in_page);
    const long dst = (long)page * page_bytes + head_bytes + (long)in_page * (kD * 2) + lane * 4;
    *(uint32_t*)(const_cast<uint8_t*>(a.k_pages) + dst) = *(const uint32_t*)(kn + lane * 4);
    *(uint32_t*)(const_cast<uint8_t*>(a.v_pages) + dst) = *(const uint32_t*)(vn + lane * 4);
  }

  __device__ inline void issue(int tile, const Pages& p, TileRegs& r) const {
    FastPager::issue(tile, p, r);
    const int rel = new_row(tile, p);
    if (rel >= 0) take_new<true>(rel, p, r);
  }
};

// Contiguous K/V [B, Hkv, N, 128] (cuh:128-178): token t of (row, kv head) at
// ((row*Hkv + kvh)*N + t)*256 bytes, N = context.  Same per-lane operand layout as the
// page-16 pager, with no block table to read.
struct ContigPager {
  struct Pages {};
  using Raw = TileRegs;
  const DecodeArgs& a;
  long base;         // byte offset of token 0 of (row, kv head)
  int lim;
  uint32_t koff[4];
  uint32_t voff[8];

  __device__ ContigPager(const DecodeArgs& args, int row, int kvh, int limit, int lane)
      : a(args), lim(limit) {
    const int hkv = a.hkv / a.kv_div;
    base = ((long)row * hkv + kvh / a.kv_div) * a.context * (kD * 2);
    const int c = lane & 15, g = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) koff[kk] = c * 256 + kk * 64 + g * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) voff[j] = (4 * g + (j & 3)) * 256 + c * 16;
  }

  __device__ inline Pages lookup(int) const { return {}; }

  __device__ inline void block_rsrc(int tile, int b, const Pages&, __amdgpu_buffer_rsrc_t& rk,
                                    __amdgpu_buffer_rsrc_t& rv) const {
    const int tok0 = tile * kTile + b * 16;
    int nvalid = lim - tok0;
    nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
    const long off = nvalid > 0 ? base + (long)tok0 * (kD * 2) : 0;
    const int nrec = uniform(nvalid * (kD * 2));
    rk = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.k_pages + off), (short)0, nrec, kRsrcWord3);
    rv = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.v_pages + off), (short)0, nrec, kRsrcWord3);
  }

  __device__ inline void issue(int tile, const Pages& p, TileRegs& r) const {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      __amdgpu_buffer_rsrc_t rk, rv;
      block_rsrc(tile, b, p, rk, rv);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) r.k[b][kk] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff[kk], 0, kKvLoadPolicy);
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[b * 4 + j] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff[b * 4 + j], 0, kKvLoadPolicy);
    }
  }
};

// A 2-byte pager (FastPager, ContigPager, AppendPager) whose K loads take whole 128-byte
// lines and go straight to LDS, for launches of few units, where what one CU streams
// bounds the launch: a lone CU streams 35-37 GB/s with the K-operand shape (16 rows x
// 64 B per instruction) and 45-56 GB/s with whole lines.  K bypasses the registers
// (buffer_load_dwordx4 ... lds: lane i of an instruction writes the 16 bytes at slab
// offset 16 i), so a wave keeps two tiles in flight with one tile's V registers more;
// V is loaded as by the base pager.
// A slab holds a tile's two 16-token blocks, 16 rows x 256 B each, with
// 16-byte column `col` of row `row` at position col ^ row: instruction j of a block
// writes rows 4j .. 4j + 3 (lane (c, g): row 4j + g, position c, so it loads column
// c ^ row; each quad of lanes still covers one aligned 64 bytes of a row), and a
// K-operand read (lane (c, g): row c, column 4kk + g) meets each LDS bank once per 16
// lanes.  tile_k of a LineTile reads the MFMA operands back one k-block at a time.
constexpr int kSlabBytes = 8192;  // one tile's two blocks of K rows

struct LineTile : TileRegs {  // k[][] unused: K is in the slab
  const uint8_t* rd;  // this lane's K-operand row in the slab: slab + 256 c
  int col;            // g ^ c: k-block kk's 16-byte column is 4 kk ^ col
  int new_row;        // appending pagers: the new token's row of the tile, or -1
  u32x4 k_new;        // ... and bytes 16 c .. +16 of its K row
};

template <class Base, int SLABS = 1>
struct Lines : Base {
  using Raw = LineTile;
  uint8_t* slab;      // this wave's SLABS x 8 KB of LDS (wave-uniform); tile t uses slab t % SLABS
  uint32_t kline[4];  // per-lane byte offsets inside a block of instruction j's K row
  int lane;

  __device__ Lines(const DecodeArgs& args, int row, int kvh, int limit, int lane_, uint8_t* s)
      : Base(args, row, kvh, limit, lane_), slab(s), lane(lane_) {
    const int c = lane_ & 15, g = lane_ >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) kline[j] = (4 * j + g) * 256 + (c ^ (4 * j + g)) * 16;
  }

  // Rows past the block's valid ones are outside the descriptor and load as 0; their
  // scores are masked in compute_tile whatever the slab holds.  With AppendPager the new
  // token's V row is taken into the registers here and its K row is loaded beside the
  // tile, to be put into the slab once the tile has landed there (ready_tile).
  __device__ inline void issue(int tile, const typename Base::Pages& p, LineTile& r) const {
    uint8_t* sb = slab + (SLABS == 2 ? (tile & 1) * kSlabBytes : 0);
    __amdgpu_buffer_rsrc_t rk[2], rv[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) this->block_rsrc(tile, b, p, rk[b], rv[b]);
    // The loads keep their program order (ready_tile counts the ones after the K rows):
    // the tile's 8 K loads, then its 8 V loads, each group after everything issued before.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk[b], (__attribute__((address_space(3))) void*)(sb + b * 4096 + j * 1024), 16, kline[j],
            0, 0, kKvLoadPolicy);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        r.v[b * 4 + j] = __builtin_amdgcn_raw_buffer_load_b128(rv[b], this->voff[b * 4 + j], 0, kKvLoadPolicy);
    r.new_row = -1;
    if constexpr (std::is_same_v<Base, AppendPager>) {
      r.new_row = this->new_row(tile, p);
      if (r.new_row >= 0) {
        r.k_new = *(const u32x4*)(this->kn + (lane & 15) * 16);
        this->template take_new<false>(r.new_row, p, r);
      }
    }
    r.rd = sb + (lane & 15) * 256;
    asm volatile("" ::: "memory");
  }
};

// Pagers that load the K-operand layout into registers need nothing before the compute.
template <class Pager, class Raw>
__device__ inline void ready_tile(const Pager&, Raw&) {}

// The tile's K rows have reached the slab once its 8 K loads are done.  Vector memory
// loads complete in order, and at least 8 were issued after them (the tile's V loads),
// 24 with two slabs (and the next tile's 16 K and V loads): at most that many
// outstanding means the K rows are in.  The V registers are waited for by the compiler
// where they are first used, after the scores.  The wait is also a compiler memory
// barrier, so the slab's reads stay below it; consumed by the tile's MFMAs, they are
// done before the slab's next loads are issued.
template <class Base, int SLABS>
__device__ inline void ready_tile(const Lines<Base, SLABS>& pg, LineTile& r) {
  const int c = pg.lane & 15, g = pg.lane >> 4;
  if constexpr (SLABS == 2) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  if (r.new_row >= 0) {  // the appended token's K row replaces what the pool held
    const int row = r.new_row & 15;
    if (g == 0) *(u32x4*)(r.rd - c * 256 + (r.new_row >> 4) * 4096 + row * 256 + (c ^ row) * 16) = r.k_new;
    asm volatile("" ::: "memory");
  }
  r.col = g ^ c;
}

// Page-16 pager over fp8 (OCP e4m3) K/V: FastPager's table reads and per-lane rows with
// 1-byte elements (a token row is 128 bytes), K in 16-byte and V in 8-byte chunks (the
// Fp8Tile layout), unpacked exactly to fp16 / bf16 just before the tile is computed.
struct Fp8Pager {
  using Pages = FastPager::Pages;
  using Raw = Fp8Tile;
  const DecodeArgs& a;
  const int32_t* trow;
  int lim;
  long head_bytes;   // kvh * ps * 128
  long page_bytes;   // Hkv * ps * 128
  uint32_t koff[2];
  uint32_t voff[8];

  __device__ Fp8Pager(const DecodeArgs& args, int row, int kvh, int limit, int lane)
      : a(args), lim(limit) {
    trow = a.block_table + (long)row * a.max_pages;
    head_bytes = (long)kvh * a.page_size * kD;
    page_bytes = (long)a.hkv * a.page_size * kD;
    const int c = lane & 15, g = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) koff[h] = c * 128 + h * 64 + g * 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) voff[j] = (4 * g + (j & 3)) * 128 + c * 8;
  }

  __device__ inline Pages lookup(int tile) const {
    Pages p;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int tok0 = (tile < 0 ? 0 : tile) * kTile + b * 16;
      int logical, in_page;
      page_of(a, tok0, logical, in_page);
      logical = logical < a.max_pages ? logical : a.max_pages - 1;
      p.page[b] = load_scalar(trow + logical);
    }
    return p;
  }

  __device__ inline void issue(int tile, const Pages& p, Fp8Tile& r) const {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int tok0 = tile * kTile + b * 16;
      int nvalid = lim - tok0;
      nvalid = nvalid < 0 ? 0 : (nvalid > 16 ? 16 : nvalid);
      int logical, in_page;
      page_of(a, tok0, logical, in_page);
      const long off = nvalid > 0
          ? (long)clamp_page(a, p.page[b]) * page_bytes + head_bytes + (long)in_page * kD : 0;
      const int nrec = uniform(nvalid * kD);
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.k_pages + off), (short)0, nrec, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(a.v_pages + off), (short)0, nrec, kRsrcWord3);
#pragma unroll
      for (int h = 0; h < 2; ++h) r.k[b][h] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff[h], 0, kKvLoadPolicy);
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[b * 4 + j] = __builtin_amdgcn_raw_buffer_load_b64(rv, voff[b * 4 + j], 0, kKvLoadPolicy);
    }
  }
};

struct GenericPager {
  struct Pages {
    long k[2];  // byte offset of this lane's K chunk per block, or -1
    long v[8];  // byte offset of this lane's V chunk per slot, or -1
  };
  using Raw = TileRegs;
  const DecodeArgs& a;
  const int32_t* trow;
  int lim;
  long head_bytes, page_bytes;
  int c, g;

  __device__ GenericPager(const DecodeArgs& args, int row, int kvh, int limit, int lane)
      : a(args), lim(limit) {
    trow = a.block_table + (long)row * a.max_pages;
    head_bytes = (long)kvh * a.page_size * (kD * 2);
    page_bytes = (long)a.hkv * a.page_size * (kD * 2);
    c = lane & 15;
    g = lane >> 4;
  }
  __device__ inline long row_offset(int token) const {
    if (token >= lim) return -1;
    int logical, in_page;
    page_of(a, token, logical, in_page);
    const int page = clamp_page(a, trow[logical]);
    return (long)page * page_bytes + head_bytes + (long)in_page * (kD * 2);
  }
  __device__ inline Pages lookup(int tile) const {
    Pages p;
    const int tok0 = tile * kTile;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const long o = row_offset(tok0 + b * 16 + c);
      p.k[b] = o < 0 ? -1 : o + g * 16;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const long o = row_offset(tok0 + v_slot_token(g, j));
      p.v[j] = o < 0 ? -1 : o + c * 16;
    }
    return p;
  }
  __device__ inline void issue(int, const Pages& p, TileRegs& r) const {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        r.k[b][kk] = p.k[b] < 0 ? z : *(const u32x4*)(a.k_pages + p.k[b] + kk * 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) r.v[j] = p.v[j] < 0 ? z : *(const u32x4*)(a.v_pages + p.v[j]);
  }
};

// ---------------------------------------------------------------------------------
// Per-wave streaming state and tile step.
//
// Lazy rescaling: probabilities are taken relative to a per-head reference m (log2
// units) that only moves when a score exceeds it by more than kSlack, so P <= 2^kSlack
// and the O/l rescale (with its cross-lane broadcast) runs on the first tile and then
// rarely.  The true running max is tracked per lane and restored in the combine, so
// partial states keep the reference's m = max score convention.
// ---------------------------------------------------------------------------------
constexpr float kSlack = 8.0f;

template <int HB>
struct WaveState {
  f32x4 o[HB][8];  // o[hb][jj][i] = O[head hb*16 + 4g + i][dim 8c + jj], relative to m
  float m[HB];     // reference max (log2 units) of head hb*16 + c, uniform over its lanes
  float mx[HB];    // lane-local true running max (log2 units)
  float l[HB];     // lane-partial sum of exp2(x - m)
};

// MFMA operands of a tile as loaded: 2-byte K/V as is, fp8 K/V unpacked where used, so
// that the K half is unpacked for QK and the V half only for PV.
template <class Elem>
__device__ inline u32x4 tile_k(const TileRegs& r, int b, int kk) { return r.k[b][kk]; }
template <class Elem>
__device__ inline u32x4 tile_k(const Fp8Tile& r, int b, int kk) {
  const u32x4 w = r.k[b][kk >> 1];
  return Elem::unpack8((kk & 1) ? u32x2{w[2], w[3]} : u32x2{w[0], w[1]});
}
template <class Elem>
__device__ inline u32x4 tile_k(const LineTile& r, int b, int kk) {
  return *(const u32x4*)(r.rd + b * 4096 + ((4 * kk) ^ r.col) * 16);
}

// V transpose for the PV product: vt[jj] holds, for dim 8c + jj, the 8 tokens of this
// lane's slots; vt[jj][q] = (slot 2q, slot 2q + 1) of dim 8c + jj.  v_perm_b32 (operands
// S0, S1, selector) writes into byte k of its result the byte of the 8-byte value S0:S1
// (S1 bytes 0-3, S0 bytes 4-7) that byte k of the selector names.
// 2-byte V: one permute per word, the low or high halves of slots 2q and 2q + 1.
template <class Elem>
__device__ inline void transpose_v(const TileRegs& r, u32x4 (&vt)[8]) {
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int w = jj >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      vt[jj][q] = __builtin_amdgcn_perm(r.v[2 * q + 1][w], r.v[2 * q][w],
                                        (jj & 1) ? 0x07060302u : 0x05040100u);
  }
}
// fp8 V: the bytes are interleaved first, t = (slot 2q dim 2m, slot 2q + 1 dim 2m, slot 2q
// dim 2m + 1, slot 2q + 1 dim 2m + 1) with dim counted from 8c, so that the conversion of
// t's low and high byte pairs yields vt[2m][q] and vt[2m + 1][q].
template <class Elem>
__device__ inline void transpose_v(const Fp8Tile& r, u32x4 (&vt)[8]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t t = __builtin_amdgcn_perm(r.v[2 * q + 1][m >> 1], r.v[2 * q][m >> 1],
                                               (m & 1) ? 0x07030602u : 0x05010400u);
      vt[2 * m][q] = Elem::template fp8_pair<false>(t);
      vt[2 * m + 1][q] = Elem::template fp8_pair<true>(t);
    }
  }
}

template <class Elem, int HB, class Tile>
__device__ inline void compute_tile(WaveState<HB>& st, const Tile& r,
                                    const u32x4 (&qf)[HB][4], int tile, int lim, int lane,
                                    float qk) {
  const int g = lane >> 4;
  u32x4 vt[8];  // transposed V (before the first PV product)
  const int tok_base = tile * kTile + 4 * g;
  const bool partial = (tile + 1) * kTile > lim;  // wave-uniform
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      s0 = Elem::mma(tile_k<Elem>(r, 0, kk), qf[hb][kk], s0);
      s1 = Elem::mma(tile_k<Elem>(r, 1, kk), qf[hb][kk], s1);
    }
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = s0[i] * qk;
      x[4 + i] = s1[i] * qk;
    }
    if (partial) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (tok_base + i >= lim) x[i] = -INFINITY;
        if (tok_base + 16 + i >= lim) x[4 + i] = -INFINITY;
      }
    }
    float lmx = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) lmx = fmaxf(lmx, x[j]);
    st.mx[hb] = fmaxf(st.mx[hb], lmx);
    if (__builtin_amdgcn_ballot_w64(lmx > st.m[hb] + kSlack) != 0) {
      const float m_new = fmaxf(st.m[hb], head_max(lmx));
      const float corr = __builtin_amdgcn_exp2f(st.m[hb] - m_new);
      st.m[hb] = m_new;
      st.l[hb] *= corr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ci = __shfl(corr, 4 * g + i);  // lane 4g + i holds head 4g + i
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) st.o[hb][jj][i] *= ci;
      }
    }
    float p[8], psum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = __builtin_amdgcn_exp2f(x[j] - st.m[hb]);
      psum += p[j];
    }
    st.l[hb] += psum;
    if (hb == 0) transpose_v<Elem>(r, vt);
    u32x4 pa;
#pragma unroll
    for (int q = 0; q < 4; ++q) pa[q] = Elem::pack2(p[2 * q], p[2 * q + 1]);
#pragma unroll
    for (int pass = 0; pass < Elem::kPasses; ++pass) {
      if (pass == 1) {  // residual of the first rounding (bf16: the rounded value is bits << 16)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          pa[q] = Elem::pack2(p[2 * q] - __builtin_bit_cast(float, pa[q] << 16),
                              p[2 * q + 1] - __builtin_bit_cast(float, pa[q] & 0xffff0000u));
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) st.o[hb][jj] = Elem::mma(pa, vt[jj], st.o[hb][jj]);
    }
  }
}

// Streams tiles [t0, t1) of one (row, kv head) into the wave state, given the block-table
// reads of tiles t0 and t0 + 1, with DEPTH tiles of K/V in flight per wave while
// block-table reads run two tiles ahead on the scalar unit.  DEPTH 1: the other waves of
// the CU hide the latency (8 waves x 16 KB per CU already saturate HBM; two tiles in
// flight per wave on top of that made the work-queue step about 7 % slower).  DEPTH 2:
// one wave per SIMD keeps the same bytes in flight (the two-head-block kernel and the
// balanced work-queue schedule).
template <class Elem, int HB, class Pager, int DEPTH = HB>
__device__ inline void stream_range_from(WaveState<HB>& st, const Pager& pg,
                                         const u32x4 (&qf)[HB][4], int t0, int t1, int lim,
                                         int lane, float qk, typename Pager::Pages pa,
                                         typename Pager::Pages pb) {
  if constexpr (DEPTH == 1) {
    typename Pager::Raw r;
    for (int t = t0; t < t1; ++t) {
      pg.issue(t, pa, r);
      pa = pb;
      pb = pg.lookup(t + 2);
      ready_tile(pg, r);
      compute_tile<Elem, HB>(st, r, qf, t, lim, lane, qk);
    }
  } else {
    // One wave per SIMD, half the waves of a CU at one block: each wave keeps two tiles
    // in flight, so the CU holds as many bytes in flight as there.  Loads of tile t1 (one
    // past the range) cover no valid rows and read nothing.
    if (t0 >= t1) return;
    typename Pager::Raw ra, rb;
    pg.issue(t0, pa, ra);
    for (int t = t0;; t += 2) {
      pg.issue(t + 1, pb, rb);
      pa = pg.lookup(t + 2);
      ready_tile(pg, ra);
      compute_tile<Elem, HB>(st, ra, qf, t, lim, lane, qk);
      if (t + 1 >= t1) break;
      pg.issue(t + 2, pa, ra);
      pb = pg.lookup(t + 3);
      ready_tile(pg, rb);
      compute_tile<Elem, HB>(st, rb, qf, t + 1, lim, lane, qk);
      if (t + 2 >= t1) break;
    }
  }
}

template <class Elem, int HB, class Pager, int DEPTH = HB>
__device__ inline void stream_range(WaveState<HB>& st, const Pager& pg, const u32x4 (&qf)[HB][4],
                                    int t0, int t1, int lim, int lane, float qk) {
  if (t0 >= t1) return;
  stream_range_from<Elem, HB, Pager, DEPTH>(st, pg, qf, t0, t1, lim, lane, qk, pg.lookup(t0),
                                            pg.lookup(t0 + 1));
}

// ---------------------------------------------------------------------------------
// Work-unit resolution.
// ---------------------------------------------------------------------------------
struct Unit {
  int row, kvh, split, tb, te, len;
  int slot_base, row_splits;  // queue mode: slot of split 0 and the row's split count
  bool valid;
};

__device__ inline int ceil_tiles(int len) { return (len + kTile - 1) / kTile; }

// Work-queue unit from a work item and its row's length and slot offsets.  The item's
// tile range is honoured as given (cuh:298-337); a negative bound stands for the
// row-local split bound of its split (cuh:330-337), and the range is clamped to the
// row's tiles (tokens past the length are masked in the reference, cuh:217-219).
// Malformed items are marked invalid (and skipped) instead of addressing outside the
// buffers.
__device__ inline Unit queue_unit(const DecodeArgs& a, int row, int kvh, int split, int tb, int te,
                                  int len, int so0, int so1) {
  Unit u;
  u.valid = true;
  u.row = row;
  u.kvh = kvh;
  u.split = split;
  u.tb = 0;
  u.te = 0;
  u.len = 0;
  u.slot_base = 0;
  u.row_splits = 1;
  if (row < 0 || row >= a.batch || kvh < 0 || kvh >= a.hkv || split < 0) {
    u.valid = false;
    return u;
  }
  u.len = clamp_length(a, len);
  u.slot_base = so0;
  u.row_splits = so1 - so0;
  const int total = ceil_tiles(u.len);
  if (split >= u.row_splits) {
    u.valid = false;
    return u;
  }
  if (tb < 0) tb = (int)(((long)total * split) / u.row_splits);
  if (te < 0) te = (int)(((long)total * (split + 1)) / u.row_splits);
  u.tb = tb;
  u.te = te > total ? total : te;
  if (u.slot_base < 0 || u.slot_base + split >= a.total_slots) u.valid = false;
  return u;
}

template <int MODE>
__device__ inline Unit resolve_unit(const DecodeArgs& a, int idx) {
  Unit u;
  u.valid = true;
  u.slot_base = 0;
  u.row_splits = 1;
  if (MODE == kDirect) {
    u.row = idx / a.hkv;
    u.kvh = idx - u.row * a.hkv;
    u.split = 0;
    u.len = row_length(a, u.row);
    u.tb = 0;
    u.te = ceil_tiles(u.len);
  } else if (MODE == kSplit) {
    const int per_row = a.hkv * a.num_splits;
    u.row = idx / per_row;
    const int rem = idx - u.row * per_row;
    u.kvh = rem / a.num_splits;
    u.split = rem - u.kvh * a.num_splits;
    u.len = row_length(a, u.row);
    const int total = ceil_tiles(u.len);
    // Row-local split bounds, cuh:330-337.
    u.tb = (int)(((long)total * u.split) / a.num_splits);
    u.te = (int)(((long)total * (u.split + 1)) / a.num_splits);
  } else {
    const int32_t* w = a.work_items + (long)idx * 5;
    const int row = load_scalar(w + 0), kvh = load_scalar(w + 1), split = load_scalar(w + 2);
    const int tb = load_scalar(w + 3), te = load_scalar(w + 4);
    const int row_c = row < 0 ? 0 : (row >= a.batch ? a.batch - 1 : row);
    u = queue_unit(a, row, kvh, split, tb, te, uniform(a.seq_lens[row_c]),
                   uniform(a.split_offsets[row_c]), uniform(a.split_offsets[row_c + 1]));
  }
  return u;
}

// ---------------------------------------------------------------------------------
// Partial-state stores and loads.  With the fused merge another workgroup (possibly on
// another XCD, behind another L2) reads the states in the same launch: they are written
// and read with agent-scope atomic accesses, and ordered by the release/acquire of the
// arrival counter (arrive).
// ---------------------------------------------------------------------------------
__device__ inline void put_f32(float* p, float v, bool coherent) {
  if (coherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}
__device__ inline void put_f32x4(float* p, f32x4 v, bool coherent) {
  if (coherent) {
    __hip_atomic_store((uint64_t*)p, __builtin_bit_cast(uint64_t, f32x2{v[0], v[1]}),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store((uint64_t*)p + 1, __builtin_bit_cast(uint64_t, f32x2{v[2], v[3]}),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *(f32x4*)p = v;
  }
}
template <bool COHERENT>
__device__ inline float get_f32(const float* p) {
  if (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}
template <bool COHERENT>
__device__ inline f32x2 get_f32x2(const float* p) {
  if (COHERENT)
    return __builtin_bit_cast(f32x2, __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT));
  return *(const f32x2*)p;
}
// Waits until every memory access this wave issued has completed.

// Neutral partial state of an empty split (cuh:340-363): m = -FLT_MAX, l = 0, acc = 0.
__device__ inline void write_neutral(const DecodeArgs& a, long state0, long state_stride,
                                     int G, int tid, int nthreads, bool coherent) {
  for (int idx = tid; idx < G * (kD / 4); idx += nthreads) {
    const int h = idx / (kD / 4), d = (idx % (kD / 4)) * 4;
    const long s = state0 + (long)h * state_stride;
    put_f32x4(a.part_acc + s * kD + d, f32x4{0.f, 0.f, 0.f, 0.f}, coherent);
    if (d == 0) {
      put_f32(a.part_m + s, -FLT_MAX, coherent);
      put_f32(a.part_l + s, 0.f, coherent);
    }
  }
}

template <class Elem>
__device__ inline void store_out4(uint8_t* out, long elem, f32x4 v) {
  u32x2 w;
  w[0] = Elem::pack2(v[0], v[1]);
  w[1] = Elem::pack2(v[2], v[3]);
  *(u32x2*)(out + elem * 2) = w;
}

// Reductions over the wave's 64 lanes with DPP (no LDS): within quads (quad_perm), half
// rows and rows (mirrors), then row 0 into row 1 and row 2 into row 3 (row_bcast:15, rows
// 1 and 3 only) and rows 0-1 into rows 2-3 (row_bcast:31, rows 2 and 3 only).  Lane 63
// then holds the result, which is returned to every lane as a scalar.  Rows left out by a
// row mask keep `ident`.
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_f32(float ident, float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ident),
                                                               __builtin_bit_cast(int, x), CTRL,
                                                               ROW_MASK, 0xf, false));
}
__device__ inline float wave_max(float x) {
  constexpr float id = -FLT_MAX;
  x = fmaxf(x, dpp_f32<0xb1, 0xf>(id, x));   // quad_perm:[1,0,3,2]
  x = fmaxf(x, dpp_f32<0x4e, 0xf>(id, x));   // quad_perm:[2,3,0,1]
  x = fmaxf(x, dpp_f32<0x141, 0xf>(id, x));  // row_half_mirror
  x = fmaxf(x, dpp_f32<0x140, 0xf>(id, x));  // row_mirror
  x = fmaxf(x, dpp_f32<0x142, 0xa>(id, x));  // row_bcast:15
  x = fmaxf(x, dpp_f32<0x143, 0xc>(id, x));  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
__device__ inline float wave_sum(float x) {
  x += dpp_f32<0xb1, 0xf>(0.f, x);
  x += dpp_f32<0x4e, 0xf>(0.f, x);
  x += dpp_f32<0x141, 0xf>(0.f, x);
  x += dpp_f32<0x140, 0xf>(0.f, x);
  x += dpp_f32<0x142, 0xa>(0.f, x);
  x += dpp_f32<0x143, 0xc>(0.f, x);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// ---------------------------------------------------------------------------------
// LSE merge of one query head's partial states by one wave (cuh:719-784): M = max m,
// L = sum e^(m - M) l, A = sum e^(m - M) acc, O = A / L (0 when L == 0).  Slot s's state
// index is base + s * stride.  In queue mode, slots of splits the builder leaves empty
// (split0 + s of nsplit splits over `total` tiles) hold no state and are skipped; the
// reference reads them uninitialised.  All loads of a chunk of up to 32 slots are
// issued together: lane s loads slot s's (m, l) and each lane its two dims of every
// slot's acc.  Lane owns output dims 2*lane, 2*lane + 1 of `out` (128 elements).
// ---------------------------------------------------------------------------------
constexpr int kMergeChunk = 32;

// Running LSE merge held by one wave; lane owns output dims 2*lane, 2*lane + 1.
struct LseAcc {
  float M = -FLT_MAX, L = 0.f;
  f32x2 A = {0.f, 0.f};

  // Folds in up to 32 states: lane j holds (ms, ls) of state j (valid when ok); v[j] holds
  // this lane's two dims of state j's acc.
  __device__ inline void fold(bool ok, float ms, float ls, const f32x2 (&v)[kMergeChunk]) {
    const float cm = wave_max(ok ? ms : -FLT_MAX);
    const float m_new = fmaxf(M, cm);
    const float corr = __builtin_amdgcn_exp2f((M - m_new) * kLog2e);
    M = m_new;
    const float w = ok ? __builtin_amdgcn_exp2f((ms - M) * kLog2e) : 0.f;
    L = L * corr + wave_sum(ok ? w * ls : 0.f);  // select: skipped slots may hold NaN
    A *= corr;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), j));
      A[0] += wj != 0.f ? wj * v[j][0] : 0.f;  // select, not multiply: skipped slots may hold NaN
      A[1] += wj != 0.f ? wj * v[j][1] : 0.f;
    }
  }

  template <class Elem>
  __device__ inline void store(uint8_t* out, int lane) const {
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *(uint32_t*)(out + 4 * lane) = Elem::pack2(A[0] * inv, A[1] * inv);
  }
};

// Up to 32 slot states as one wave loads them: lane j holds (m, l) of slot c0 + j and
// v[j] this lane's two dims of that slot's acc.  All loads are issued together; the acc
// of slots past the chunk (n, uniform) is not loaded (v[j] = 0, and fold gives those
// slots weight 0), since a merge of many short rows would otherwise spend most of its
// time re-reading the last state.
struct SlotChunk {
  float ms, ls;
  f32x2 v[kMergeChunk];
};

template <bool COHERENT>
__device__ inline void load_chunk(SlotChunk& c, const float* pm, const float* pl, const float* pacc,
                                  long base, long stride, int c0, int n, int lane) {
  n = uniform(n);
  const int s_lane = c0 + (lane < n ? lane : n - 1);
  c.ms = get_f32<COHERENT>(pm + base + (long)s_lane * stride);
  c.ls = get_f32<COHERENT>(pl + base + (long)s_lane * stride);
#pragma unroll
  for (int j = 0; j < kMergeChunk; ++j)
    c.v[j] = j < n ? get_f32x2<COHERENT>(pacc + (base + (long)(c0 + j) * stride) * kD + 2 * lane)
                   : f32x2{0.f, 0.f};
}

// load_chunk through buffer descriptors that cover the chunk's states (n >= 1): when
// `enable` is false they cover nothing, and the loads return zeros without reading memory.
__device__ inline void load_chunk_if(SlotChunk& c, const float* pm, const float* pl, const float* pacc,
                                     long base, long stride, int n, int lane, bool enable) {
  n = uniform(n);
  const int span = enable ? (int)((long)(n - 1) * stride + 1) : 0;  // states from base
  const __amdgpu_buffer_rsrc_t rm =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(pm + base), (short)0, uniform(span * 4), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rl =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(pl + base), (short)0, uniform(span * 4), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(pacc + base * kD), (short)0, uniform(span * kD * 4), kRsrcWord3);
  const int s_lane = lane < n ? lane : n - 1;
  c.ms = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, (int)(s_lane * stride * 4), 0, 0));
  c.ls = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, (int)(s_lane * stride * 4), 0, 0));
#pragma unroll
  for (int j = 0; j < kMergeChunk; ++j)
    c.v[j] = j < n ? __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   ra, (int)((j * stride * kD + 2 * lane) * 4), 0, 0))
                   : f32x2{0.f, 0.f};
}

// Whether slot s of a row holds a state.  In queue mode the builder leaves splits with no
// tiles unwritten (split0 + s of nsplit splits over `total` tiles); `all` (a queue that
// writes every slot, see queue_writes_every_slot) folds every slot, as the reference does.
template <bool QUEUE>
__device__ inline bool slot_live(int s, int count, long total, int nsplit, int split0,
                                 bool all = false) {
  // With at least as many tiles as splits every split holds one (the divisions are
  // skipped: total and nsplit are wave-uniform).
  return s < count && (all || !(QUEUE && total < nsplit &&
                                total * (split0 + s) / nsplit == total * (split0 + s + 1) / nsplit));
}

// Whether a work queue writes every slot of its rows: the reference merges every slot of
// a row (cuh:753-784), so a queue it defines has one item per (slot, kv head), i.e. at
// least Hkv x (split_offsets[B] - split_offsets[0]) items.  The builder's queues emit no
// item for a split without tiles (benchmark_serving_trace.py:699-700), leaving those slots
// unwritten (the reference then merges uninitialised memory); with fewer items the merge
// therefore skips the slots whose row-local bounds are empty and folds the rest.
__device__ inline bool queue_writes_every_slot(long num_tasks, int hkv, int so_first, int so_last) {
  return num_tasks >= (long)hkv * ((long)so_last - so_first);
}

// Folds slot states [c_begin, count) into acc, 32 at a time.
template <bool QUEUE, bool COHERENT>
__device__ inline void fold_slots(LseAcc& acc, const float* pm, const float* pl, const float* pacc,
                                  long base, long stride, int count, long total, int nsplit,
                                  int split0, int lane, int c_begin = 0, bool all = false) {
  for (int c0 = c_begin; c0 < count; c0 += kMergeChunk) {
    const int n = count - c0 < kMergeChunk ? count - c0 : kMergeChunk;
    SlotChunk c;
    load_chunk<COHERENT>(c, pm, pl, pacc, base, stride, c0, n, lane);
    acc.fold(lane < n && slot_live<QUEUE>(c0 + lane, count, total, nsplit, split0, all), c.ms,
             c.ls, c.v);
  }
}

// fold_slots with the next chunk's loads in flight while a chunk is folded, so that a long
// range costs about one memory round trip instead of one per chunk.
template <bool QUEUE>
__device__ inline void fold_slots_pipelined(LseAcc& acc, const float* pm, const float* pl,
                                            const float* pacc, long base, long stride, int count,
                                            long total, int nsplit, int split0, int lane) {
  if (count <= 0) return;
  SlotChunk cur, nxt;
  load_chunk<false>(cur, pm, pl, pacc, base, stride, 0, count < kMergeChunk ? count : kMergeChunk,
                    lane);
  for (int c0 = 0; c0 < count; c0 += kMergeChunk) {
    const int n = count - c0 < kMergeChunk ? count - c0 : kMergeChunk;
    const int c1 = c0 + kMergeChunk;
    if (c1 < count)
      load_chunk<false>(nxt, pm, pl, pacc, base, stride, c1,
                        count - c1 < kMergeChunk ? count - c1 : kMergeChunk, lane);
    acc.fold(lane < n && slot_live<QUEUE>(c0 + lane, count, total, nsplit, split0), cur.ms, cur.ls,
             cur.v);
    cur = nxt;
  }
}

// Wide fold of up to kWideStates states of one query head by one wave, every load in
// flight at once (one memory round trip; a wave tracks at most 63 vector loads, so the
// 8-byte loads of fold_slots fit 32 states per round trip).  Lanes 0-31 load the even
// states and lanes 32-63 the odd ones with 16-byte loads (4 dims per lane): 2 states per
// load.  Lane j holds (m, l) of states j and j + 64.  Each half accumulates its states;
// the halves are added and the result is returned in the LseAcc layout (lane owns dims
// 2 lane, 2 lane + 1).  States are base + s * stride, s < n (wave-uniform, 1 <= n <=
// kWideStates); in queue mode, slots of empty splits are skipped as in fold_slots.
constexpr int kWideLoads = 56;
constexpr int kWideStates = 2 * kWideLoads;

__device__ inline void fold_wide(LseAcc& acc, const float* pm, const float* pl, const float* pacc,
                                 long base, long stride, int n, long total, int nsplit,
                                 int split0, int lane) {
  n = uniform(n);
  const int half = lane >> 5, q = lane & 31;
  const int s0 = lane < n ? lane : n - 1, s1 = lane + 64 < n ? lane + 64 : n - 1;
  const float m0 = pm[base + (long)s0 * stride], l0 = pl[base + (long)s0 * stride];
  const float m1 = pm[base + (long)s1 * stride], l1 = pl[base + (long)s1 * stride];
  f32x4 v[kWideLoads];
#pragma unroll
  for (int i = 0; i < kWideLoads; ++i) {
    const int st = 2 * i + half < n ? 2 * i + half : n - 1;
    v[i] = 2 * i < n ? *(const f32x4*)(pacc + (base + (long)st * stride) * kD + 4 * q)
                     : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bool ok0 = lane < n && slot_live<true>(lane, n, total, nsplit, split0);
  const bool ok1 = lane + 64 < n && slot_live<true>(lane + 64, n, total, nsplit, split0);
  const float M = wave_max(fmaxf(ok0 ? m0 : -FLT_MAX, ok1 ? m1 : -FLT_MAX));
  const float w0 = ok0 ? __builtin_amdgcn_exp2f((m0 - M) * kLog2e) : 0.f;
  const float w1 = ok1 ? __builtin_amdgcn_exp2f((m1 - M) * kLog2e) : 0.f;
  const float L = wave_sum((ok0 ? w0 * l0 : 0.f) + (ok1 ? w1 * l1 : 0.f));  // skipped slots may hold NaN
  f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kWideLoads; ++i) {
    if (2 * i >= n) break;
    const float src_e = 2 * i < 64 ? w0 : w1, src_o = 2 * i + 1 < 64 ? w0 : w1;
    const float we = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, src_e), (2 * i) & 63));
    const float wo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, src_o), (2 * i + 1) & 63));
    const float w = half ? wo : we;
#pragma unroll
    for (int k = 0; k < 4; ++k) A[k] += w != 0.f ? w * v[i][k] : 0.f;  // select: unused slots may hold NaN
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) A[k] += __shfl_xor(A[k], 32);
  // Lane j's dims 2j, 2j + 1 sit in lane j / 2 (components 0-1 or 2-3).
  const int src = (lane >> 1) & 31;
  const float x0 = __shfl(A[0], src), x1 = __shfl(A[1], src);
  const float x2 = __shfl(A[2], src), x3 = __shfl(A[3], src);
  acc.M = M;
  acc.L = L;
  acc.A = (lane & 1) ? f32x2{x2, x3} : f32x2{x0, x1};
}

// Fused merge of query head qh of a work-queue row by one wave, run by the last work item
// of the row's (row, kv head) group to finish (cuh:648-716).  Slots are
// (split_offsets[row] + s)*Hq + qh.
__device__ inline int unit_slot_count(const DecodeArgs& a, const Unit& u) {
  return u.slot_base + u.row_splits > a.total_slots ? a.total_slots - u.slot_base : u.row_splits;
}

// `all`: the queue writes every slot (queue_writes_every_slot).
template <class Elem>
__device__ inline void fused_merge_head(const DecodeArgs& a, const Unit& u, int qh, int lane,
                                        bool all) {
  const int out_row = a.out_indices ? a.out_indices[u.row] : u.row;
  if (out_row < 0 || out_row >= a.out_rows) return;
  LseAcc acc;
  fold_slots<true, true>(acc, a.part_m, a.part_l, a.part_acc, (long)u.slot_base * a.hq + qh, a.hq,
                         unit_slot_count(a, u), ceil_tiles(u.len), u.row_splits, 0, lane, 0, all);
  acc.store<Elem>(a.out + ((long)out_row * a.hq + qh) * kD * 2, lane);
}

// Work items of one (row, kv head): one per slot of the row when the queue writes every
// slot (the reference's count, row_splits, cuh:659), else one per non-empty split (the
// builder emits no empty ones), min(S_row, T).
__device__ inline int expected_arrivals(const DecodeArgs& a, const Unit& u, bool all) {
  if (all) return unit_slot_count(a, u);
  const int total = ceil_tiles(u.len);
  return u.row_splits < total ? u.row_splits : total;
}

// Arrival of a unit whose partial states are written: the last unit of its (row, kv head)
// merges the group's G heads and clears the counter.  With `nwaves` > 1 the whole
// workgroup calls this (it synchronises); with 1, a single wave.
//
// Ordering, by the memory model: the workgroup's state stores happen before the barrier
// (with one wave, its lanes issue in lock step, which the AMDGPU memory model treats as
// ordered at wavefront scope); wave 0's lane 0 counts the arrival with an agent-scope
// release read-modify-write, which releases those stores to every other unit of the
// group.  The arrivals' RMWs form one release sequence on the counter, so the last
// arrival, which reads the value the others' RMWs left, synchronises with every one of
// them through an agent-scope acquire fence after its RMW; only it pays for the acquire
// (an L2 invalidate), the others only for the release.  The second barrier passes the
// acquire on to the merging waves.
template <class Elem>
__device__ inline void arrive(const DecodeArgs& a, const Unit& u, int qh0, int lane, int wave,
                              int nwaves, bool all) {
  __shared__ int last_flag;
  int32_t* counter = a.merge_counters + (long)u.row * a.hkv + u.kvh;
  if (nwaves > 1) __syncthreads();
  int last = 0;
  if (wave == 0 && lane == 0) {
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    last = old == expected_arrivals(a, u, all) - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (nwaves > 1) last_flag = last;
  }
  if (nwaves > 1) {
    __syncthreads();
    last = last_flag;
  } else {
    last = uniform(last);
  }
  if (last) {
    for (int h = wave; h < a.group; h += nwaves) fused_merge_head<Elem>(a, u, qh0 + h, lane, all);
    if (wave == 0 && lane == 0)
      __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------------
// Pieces shared by the two decode paths.
// ---------------------------------------------------------------------------------
// Partial-state addressing: state index of head h is state0 + h * stride.
template <int MODE>
__device__ inline void unit_states(const DecodeArgs& a, const Unit& u, int qh0, long& state0,
                                   long& stride) {
  state0 = 0;
  stride = 1;
  if (MODE == kSplit) {
    state0 = ((long)u.row * a.hq + qh0) * a.num_splits + u.split;
    stride = a.num_splits;
  } else if (MODE == kQueue) {
    state0 = (long)(u.slot_base + u.split) * a.hq + qh0;
  }
}

// Q^T operand: lane (g, c) holds head hb*16 + c, dims 32kk + 8g .. +8 (with K16, for fp8
// K, dims 64(kk/2) + 16g + 8(kk%2) .. +8, matching Fp8Tile's K layout).  The query row is
// `row`, or `q_loaded` (q_indices[row], the same in every lane) when q_indices is set.
// q_loaded may still be in flight: the address is formed per lane, so its wait falls
// right before the Q loads.
template <int HB, bool K16 = false>
__device__ inline void load_q(const DecodeArgs& a, int q_loaded, int row, int qh0, int lane,
                              u32x4 (&qf)[HB][4]) {
  const int c = lane & 15, g = lane >> 4;
  int q_row = a.q_indices ? q_loaded : row;
  q_row = q_row < 0 ? 0 : (q_row >= a.q_rows ? a.q_rows - 1 : q_row);
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int h = hb * 16 + c;
    const uint8_t* qp = a.q + (((long)q_row * a.hq + qh0 + h) * kD + (K16 ? 16 : 8) * g) * 2;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      const int off = K16 ? (64 * (kk >> 1) + 8 * (kk & 1)) * 2 : kk * 64;
      qf[hb][kk] = h < a.group ? *(const u32x4*)(qp + off) : z;
    }
  }
}

template <int HB>
__device__ inline void init_state(WaveState<HB>& st) {
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    st.m[hb] = -FLT_MAX;
    st.mx[hb] = -FLT_MAX;
    st.l[hb] = 0.f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) st.o[hb][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// K/V addressing of a launch: paged with 16-token-aligned pages, paged with any page
// size, or contiguous.
// kPgLines, kPgContigLines and kPgAppendLines are kPgFast, kPgContig and kPgAppend with
// whole-line K loads (Lines).
enum : int { kPgGeneric = 0, kPgFast = 1, kPgContig = 2, kPgFp8 = 3, kPgAppend = 4, kPgLines = 5,
             kPgContigLines = 6, kPgAppendLines = 7 };

// Streams tiles [t0, t1) of (row, kvh) into the wave state without finishing it, so that
// several ranges can be streamed into one state (finish_state ends it).  `slab` is the
// wave's 8 KB of LDS for the whole-line pagers.
template <class Elem, int HB, int PG, int DEPTH = HB>
__device__ inline void stream_tiles(const DecodeArgs& a, WaveState<HB>& st, const u32x4 (&qf)[HB][4],
                                    int row, int kvh, int t0, int t1, int len, int lane,
                                    bool have_first = false, FastPager::Pages f0 = {},
                                    FastPager::Pages f1 = {}, uint8_t* slab = nullptr) {
  const long lim_l = (long)t1 * kTile;
  const int lim = uniform(lim_l < len ? (int)lim_l : len);
  const float qk = a.score_scale;
  if constexpr (PG == kPgLines || PG == kPgContigLines || PG == kPgAppendLines) {
    using Base = std::conditional_t<PG == kPgLines, FastPager,
                                    std::conditional_t<PG == kPgContigLines, ContigPager, AppendPager>>;
    Lines<Base, DEPTH> pg(a, row, kvh, lim, lane, slab);
    stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
    // The loop's last loads (the tile after the range, which reads nothing) still write
    // the slab; they are done before the LDS is used for the combine or the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else if constexpr (PG == kPgFast) {
    FastPager pg(a, row, kvh, lim, lane);
    if (have_first) stream_range_from<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk, f0, f1);
    else stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
  } else if constexpr (PG == kPgAppend) {
    AppendPager pg(a, row, kvh, lim, lane);
    if (have_first) stream_range_from<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk, f0, f1);
    else stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
  } else if constexpr (PG == kPgFp8) {
    Fp8Pager pg(a, row, kvh, lim, lane);
    if (have_first) stream_range_from<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk, f0, f1);
    else stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
  } else if constexpr (PG == kPgContig) {
    ContigPager pg(a, row, kvh, lim, lane);
    stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
  } else {
    GenericPager pg(a, row, kvh, lim, lane);
    stream_range<Elem, HB, decltype(pg), DEPTH>(st, pg, qf, t0, t1, lim, lane, qk);
  }
}

// Ends a wave state: the lane-partial sums and maxima of each head are reduced over the
// head's four lanes.
template <int HB>
__device__ inline void finish_state(WaveState<HB>& st) {
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    st.l[hb] = head_sum(st.l[hb]);
    st.mx[hb] = head_max(st.mx[hb]);
  }
}

template <class Elem, int HB, int PG, int DEPTH = HB>
__device__ inline void stream_unit(const DecodeArgs& a, WaveState<HB>& st, const u32x4 (&qf)[HB][4],
                                   int row, int kvh, int t0, int t1, int len, int lane,
                                   bool have_first = false, FastPager::Pages f0 = {},
                                   FastPager::Pages f1 = {}, uint8_t* slab = nullptr) {
  stream_tiles<Elem, HB, PG, DEPTH>(a, st, qf, row, kvh, t0, t1, len, lane, have_first, f0, f1,
                                    slab);
  finish_state<HB>(st);
}

// ---------------------------------------------------------------------------------
// Writers of a unit's final state.  `Dest` addresses partial states: head h of the unit
// goes to state index state0 + h * stride of (m, l, acc); `coherent` selects agent-scope
// stores (fused merge).  Direct launches write the normalised output instead.
// ---------------------------------------------------------------------------------
struct Dest {
  float* m;
  float* l;
  float* acc;
  long state0, stride;
  bool coherent;
};

// One wave's state is the unit's whole state: write it from registers.  Lanes (*, c) hold
// the softmax state of head hb*16 + c; lane (g, c) holds O of heads hb*16 + 4g + i, dims
// 8c .. 8c + 7.
template <class Elem, int HB, bool DIRECT>
__device__ inline void write_wave_state(const DecodeArgs& a, const WaveState<HB>& st, int qh0,
                                        int out_row, const Dest& d, int lane) {
  const int G = a.group, c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    // Partial states relative to the true max (m = max score, l = sum exp(s - m),
    // acc = sum exp(s - m) v; cuh:620-632); the direct op normalises instead.
    const float rescale = __builtin_amdgcn_exp2f(st.m[hb] - st.mx[hb]);
    const float inv_l = st.l[hb] > 0.f ? 1.f / st.l[hb] : 0.f;
    if (!DIRECT && g == 0 && hb * 16 + c < G) {
      const long s = d.state0 + (long)(hb * 16 + c) * d.stride;
      put_f32(d.m + s, st.mx[hb] * kLn2, d.coherent);
      put_f32(d.l + s, st.l[hb] * rescale, d.coherent);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = hb * 16 + 4 * g + i;  // lane 4g + i holds the state of head h
      const float r = __shfl(DIRECT ? inv_l : rescale, 4 * g + i) * a.v_scale;
      const f32x4 lo = f32x4{st.o[hb][0][i], st.o[hb][1][i], st.o[hb][2][i], st.o[hb][3][i]} * r;
      const f32x4 hi = f32x4{st.o[hb][4][i], st.o[hb][5][i], st.o[hb][6][i], st.o[hb][7][i]} * r;
      if (h >= G) continue;
      if (DIRECT) {
        if (out_row >= 0 && out_row < a.out_rows) {
          const long e = ((long)out_row * a.hq + qh0 + h) * kD + 8 * c;
          store_out4<Elem>(a.out, e, lo);
          store_out4<Elem>(a.out, e + 4, hi);
        }
      } else {
        float* dst = d.acc + (d.state0 + (long)h * d.stride) * kD + 8 * c;
        put_f32x4(dst, lo, d.coherent);
        put_f32x4(dst + 4, hi, d.coherent);
      }
    }
  }
}

// Combines the NW waves' states of one unit through LDS, one chunk of heads at a time
// (16 heads with 4 waves, 8 with 8, so the O staging stays at 32 KB), and writes the
// result.  LDS: m[w][32] (reference max), l[w][32], x[w][32] (true max),
// o[w][gh][128] with gh = min(G, chunk).  Starts with a barrier, so LDS can be reused by
// consecutive units of one workgroup.
template <class Elem, int HB, int NW, bool DIRECT>
__device__ inline void combine_waves(const DecodeArgs& a, const WaveState<HB>& st, float* lds,
                                     int qh0, int out_row, const Dest& d, int tid, int lane,
                                     int wave) {
  constexpr int kThreads = NW * 64;
  constexpr int kChunk = NW == 8 ? 8 : 16;
  const int G = a.group, c = lane & 15, g = lane >> 4;
  const int gh = G < kChunk ? G : kChunk;
  float* sm_m = lds;
  float* sm_l = lds + NW * 32;
  float* sm_x = lds + 2 * NW * 32;
  float* sm_o = lds + 3 * NW * 32;
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int h = hb * 16 + c;
      if (h < G) {
        sm_m[wave * 32 + h] = st.m[hb];
        sm_l[wave * 32 + h] = st.l[hb];
        sm_x[wave * 32 + h] = st.mx[hb];
      }
    }
  }
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
#pragma unroll
    for (int sub = 0; sub < 16 / kChunk; ++sub) {
      const int h0 = hb * 16 + sub * kChunk;
      const int nh = G - h0 < kChunk ? G - h0 : kChunk;
      if (nh <= 0) break;
      if (hb > 0 || sub > 0) __syncthreads();  // previous chunk's readers are done with sm_o
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int hh = 4 * g + i - sub * kChunk;
        if (hh >= 0 && hh < nh) {
          float* dst = sm_o + ((long)wave * gh + hh) * kD + 8 * c;
          *(f32x4*)dst = f32x4{st.o[hb][0][i], st.o[hb][1][i], st.o[hb][2][i], st.o[hb][3][i]};
          *(f32x4*)(dst + 4) = f32x4{st.o[hb][4][i], st.o[hb][5][i], st.o[hb][6][i], st.o[hb][7][i]};
        }
      }
      __syncthreads();
      for (int idx = tid; idx < nh * (kD / 4); idx += kThreads) {
        const int hh = idx / (kD / 4), dd = (idx % (kD / 4)) * 4;
        const int h = h0 + hh;
        float M = -FLT_MAX;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w * 32 + h]);
        float L = 0.f;
        f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float e = __builtin_amdgcn_exp2f(sm_m[w * 32 + h] - M);
          L += e * sm_l[w * 32 + h];
          A += e * *(const f32x4*)(sm_o + ((long)w * gh + hh) * kD + dd);
        }
        if (DIRECT) {
          if (out_row >= 0 && out_row < a.out_rows) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            store_out4<Elem>(a.out, ((long)out_row * a.hq + qh0 + h) * kD + dd, A * (inv * a.v_scale));
          }
        } else {
          // Re-express (L, A) relative to the true max so the partial state is
          // (m = max score, l = sum exp(s - m), acc = sum exp(s - m) v) as in cuh:620-632.
          float Mx = -FLT_MAX;
#pragma unroll
          for (int w = 0; w < NW; ++w) Mx = fmaxf(Mx, sm_x[w * 32 + h]);
          const float rescale = __builtin_amdgcn_exp2f(M - Mx);
          const long s = d.state0 + (long)h * d.stride;
          put_f32x4(d.acc + s * kD + dd, A * (rescale * a.v_scale), d.coherent);
          if (dd == 0) {
            put_f32(d.m + s, Mx * kLn2, d.coherent);
            put_f32(d.l + s, L * rescale, d.coherent);
          }
        }
      }
    }
  }
}

// Combines the NW waves' states of one unit without a barrier.  Each wave stores its state
// in LDS and counts itself in `arrivals`; the last wave to arrive combines all NW states
// and writes the result, and the others return at once.  Waves of one unit finish up to a
// tile's memory round trip apart; the early ones free their slots for the CU's next
// workgroup, which starts its own loads instead of waiting at a barrier.  LDS:
// m[w][32] (reference max), l[w][32], x[w][32] (true max), o[w][G][128].  `arrivals`
// is zero when the unit starts.  Returns true in the wave that wrote the result.
template <class Elem, int HB, int NW, bool DIRECT>
__device__ inline bool combine_async(const DecodeArgs& a, const WaveState<HB>& st, float* lds,
                                     int* arrivals, int qh0, int out_row, const Dest& d, int lane,
                                     int wave) {
  const int G = a.group, c = lane & 15, g = lane >> 4;
  float* sm_m = lds;
  float* sm_l = lds + NW * 32;
  float* sm_x = lds + 2 * NW * 32;
  float* sm_o = lds + 3 * NW * 32;
  if (g == 0) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int h = hb * 16 + c;
      if (h < G) {
        sm_m[wave * 32 + h] = st.m[hb];
        sm_l[wave * 32 + h] = st.l[hb];
        sm_x[wave * 32 + h] = st.mx[hb];
      }
    }
  }
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = hb * 16 + 4 * g + i;
      if (h < G) {
        float* dst = sm_o + ((long)wave * G + h) * kD + 8 * c;
        *(f32x4*)dst = f32x4{st.o[hb][0][i], st.o[hb][1][i], st.o[hb][2][i], st.o[hb][3][i]};
        *(f32x4*)(dst + 4) = f32x4{st.o[hb][4][i], st.o[hb][5][i], st.o[hb][6][i], st.o[hb][7][i]};
      }
    }
  }
  // Publish this wave's LDS stores, then count the wave (the fences order the whole
  // wave's LDS accesses around lane 0's atomic).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  int before = 0;
  if (lane == 0) before = __hip_atomic_fetch_add(arrivals, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (uniform(before) != NW - 1) return false;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int idx = lane; idx < G * (kD / 4); idx += 64) {
    const int h = idx / (kD / 4), dd = (idx % (kD / 4)) * 4;
    float M = -FLT_MAX;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm_m[w * 32 + h]);
    float L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float e = __builtin_amdgcn_exp2f(sm_m[w * 32 + h] - M);
      L += e * sm_l[w * 32 + h];
      A += e * *(const f32x4*)(sm_o + ((long)w * G + h) * kD + dd);
    }
    if (DIRECT) {
      if (out_row >= 0 && out_row < a.out_rows) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        store_out4<Elem>(a.out, ((long)out_row * a.hq + qh0 + h) * kD + dd, A * (inv * a.v_scale));
      }
    } else {
      // (L, A) re-expressed relative to the true max, as in combine_waves.
      float Mx = -FLT_MAX;
#pragma unroll
      for (int w = 0; w < NW; ++w) Mx = fmaxf(Mx, sm_x[w * 32 + h]);
      const float rescale = __builtin_amdgcn_exp2f(M - Mx);
      const long s = d.state0 + (long)h * d.stride;
      put_f32x4(d.acc + s * kD + dd, A * (rescale * a.v_scale), d.coherent);
      if (dd == 0) {
        put_f32(d.m + s, Mx * kLn2, d.coherent);
        put_f32(d.l + s, L * rescale, d.coherent);
      }
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------
// Small units (at most kSoloTiles tiles) are streamed by one wave alone: its state is
// final, so it goes straight from registers to its destination without the LDS combine.
// ---------------------------------------------------------------------------------
constexpr int kSoloTiles = 2;

template <class Elem, int HB, int PG, int MODE, int DEPTH = HB, bool FUSED = false>
__device__ void solo_unit(const DecodeArgs& a, const Unit& u, int q_loaded, int t0, int t1,
                          const Dest& d, int lane, bool have_first, FastPager::Pages f0,
                          FastPager::Pages f1, bool fused_all, uint8_t* slab = nullptr) {
  const int qh0 = u.kvh * a.group;
  u32x4 qf[HB][4];
  load_q<HB, PG == kPgFp8>(a, q_loaded, u.row, qh0, lane, qf);
  WaveState<HB> st;
  init_state<HB>(st);
  stream_unit<Elem, HB, PG, DEPTH>(a, st, qf, u.row, u.kvh, t0, t1, u.len, lane, have_first, f0,
                                   f1, slab);
  const int out_row = MODE == kDirect ? (a.out_indices ? a.out_indices[u.row] : u.row) : 0;
  write_wave_state<Elem, HB, MODE == kDirect>(a, st, qh0, out_row, d, lane);
  if constexpr (MODE == kQueue && FUSED) arrive<Elem>(a, u, qh0, lane, 0, 1, fused_all);
}

// ---------------------------------------------------------------------------------
// The decode kernel: one workgroup per unit.
// ---------------------------------------------------------------------------------
// Register budget: G <= 16 (one head block) must fit two waves per SIMD (<= 256 registers
// each); G <= 32 doubles the accumulators and may use the whole register file.
//
// ASYNC selects the barrier-free combine (combine_async) for multi-wave units; it pays
// when the launch has several units per CU, whose next workgroup then starts early.
// With the fused merge, the last work item of a (row, kv head) to finish writes that part
// of the row's output, and a row without tokens has no work items (as the builder emits
// them): its output, 0 by the merges' L == 0 rule, is written here instead, rows strided
// over the grid.  No work item writes such a row, so nothing races with these stores.
template <class Elem>
__device__ inline void zero_empty_rows(const DecodeArgs& a, int tid, int threads) {
  for (int r = blockIdx.x; r < a.batch; r += gridDim.x) {
    if (row_length(a, r) > 0) continue;
    const int out_row = a.out_indices ? a.out_indices[r] : r;
    if (out_row < 0 || out_row >= a.out_rows) continue;
    uint32_t* o = (uint32_t*)(a.out + (long)out_row * a.hq * kD * 2);
    for (int i = tid; i < a.hq * kD / 2; i += threads) o[i] = 0u;  // +0 in fp16 and bf16
  }
}

template <class Elem, int HB, int PG, int MODE, int NW, bool ASYNC, int DEPTH = HB, bool FUSED = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu((HB == 1 && DEPTH == 1) ? 2 : 1)))
void decode_kernel(DecodeArgs a) {
  constexpr int kWaves = NW;
  constexpr int kThreads = NW * 64;
  constexpr bool kLines = PG == kPgLines || PG == kPgContigLines || PG == kPgAppendLines;
  // The whole-line pagers' slabs share the LDS with the combine, which starts with a
  // barrier; the barrier-free combine would write it while other waves still stream.
  static_assert(!(kLines && ASYNC), "whole-line K needs the barrier combine");
  extern __shared__ float lds[];
  __shared__ int arrivals;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int G = a.group;
  // Fused merge: whether the queue writes every slot (the arrival count and the merge's
  // slot rule follow from it).  Loaded here, waited for at the arrival.
  int so_first = 0, so_last = 0;
  if constexpr (MODE == kQueue && FUSED) {
    so_first = load_vector_deferred(a.split_offsets);
    so_last = load_vector_deferred(a.split_offsets + a.batch);
    zero_empty_rows<Elem>(a, tid, kThreads);
  }

  // Work-queue units: one dependent round trip for the work item, then one for all it
  // points to, issued together: the row's length, slot offsets and query row (vector
  // loads, waited for together) and this wave's first two block-table reads (scalar
  // loads).  Q and the first K/V tile are issued after that, so the chain before the
  // first K/V request is two round trips.
  FastPager::Pages first0 = {}, first1 = {};
  int first_tile = -1;
  Unit u;
  int q_loaded = 0;  // q_indices[row] when q_indices is set, left in a VGPR (see load_q)
  if constexpr (MODE == kQueue && PG != kPgGeneric && PG != kPgContig) {
    const int32_t* w = a.work_items + (long)blockIdx.x * 5;
    const int row = load_scalar(w + 0), kvh = load_scalar(w + 1), split = load_scalar(w + 2);
    const int tb = load_scalar(w + 3), te = load_scalar(w + 4);
    const int row_c = row < 0 ? 0 : (row >= a.batch ? a.batch - 1 : row);
    const int kvh_c = kvh < 0 ? 0 : (kvh >= a.hkv ? a.hkv - 1 : kvh);
    const int len_l = load_vector_deferred(a.seq_lens + row_c);
    const int so0_l = load_vector_deferred(a.split_offsets + row_c);
    const int so1_l = load_vector_deferred(a.split_offsets + row_c + 1);
    const int qi_l = load_vector_deferred(a.q_indices ? a.q_indices + row_c : nullptr);
    const int n = te > tb ? te - tb : 0;
    first_tile = uniform(tb + (n * wave) / kWaves);
    const FastPager pg(a, row_c, kvh_c, 0, lane);
    first0 = pg.lookup(first_tile);
    first1 = pg.lookup(first_tile + 1);
    u = queue_unit(a, row, kvh, split, tb, te, uniform(len_l), uniform(so0_l), uniform(so1_l));
    q_loaded = uniform(qi_l);
  } else if constexpr (MODE != kQueue) {
    // The row follows from the workgroup index: its query row is requested (vector load,
    // waited for only by the Q loads) before its length (scalar load) is read.
    const int row = MODE == kDirect ? (int)blockIdx.x / a.hkv : (int)blockIdx.x / (a.hkv * a.num_splits);
    q_loaded = load_vector_lanes(a.q_indices ? a.q_indices + row : nullptr,
                                 a.batch < 0 ? lane : 0);  // batch >= 0 (checked on the host)
    u = resolve_unit<MODE>(a, blockIdx.x);
  } else {
    u = resolve_unit<MODE>(a, blockIdx.x);
    if (a.q_indices && u.valid) q_loaded = a.q_indices[u.row];
  }
  if (!u.valid) return;
  const int qh0 = u.kvh * G;
  long state0, state_stride;
  unit_states<MODE>(a, u, qh0, state0, state_stride);
  constexpr bool fused = MODE == kQueue && FUSED;
  const bool fused_all =
      fused && queue_writes_every_slot(a.num_tasks, a.hkv, uniform(so_first), uniform(so_last));
  const Dest d{a.part_m, a.part_l, a.part_acc, state0, state_stride, fused};

  if (MODE != kDirect && u.tb >= u.te) {
    write_neutral(a, state0, state_stride, G, tid, kThreads, fused);
    // An item without tiles is one of its row's arrivals too (a queue that writes every
    // slot; the builder emits none).
    if constexpr (fused) arrive<Elem>(a, u, qh0, lane, wave, kWaves, fused_all);
    return;
  }

  // Small units: wave 0 alone; the other waves return at once and free their slots for
  // the next workgroup on the CU.  No barrier is reached on this path.
  const int n = u.te - u.tb;
  if (n <= kSoloTiles) {
    if (wave == 0)
      solo_unit<Elem, HB, PG, MODE, DEPTH, FUSED>(a, u, q_loaded, u.tb, u.te, d, lane,
                                           u.tb == first_tile, first0, first1, fused_all,
                                           (uint8_t*)lds);
    return;
  }

  if constexpr (ASYNC) {
    if (tid == 0) arrivals = 0;
    __syncthreads();
  }
  u32x4 qf[HB][4];
  load_q<HB, PG == kPgFp8>(a, q_loaded, u.row, qh0, lane, qf);
  WaveState<HB> st;
  init_state<HB>(st);

  // Contiguous sub-range of the unit's tiles for this wave.
  const int w0 = uniform(u.tb + (n * wave) / kWaves);
  const int w1 = uniform(u.tb + (n * (wave + 1)) / kWaves);
  stream_unit<Elem, HB, PG, DEPTH>(a, st, qf, u.row, u.kvh, w0, w1, u.len, lane,
                                   w0 == first_tile, first0, first1,
                                   (uint8_t*)lds + (kLines ? wave * DEPTH * kSlabBytes : 0));
  const int out_row = MODE == kDirect ? (a.out_indices ? a.out_indices[u.row] : u.row) : 0;
  if constexpr (ASYNC) {
    if (!combine_async<Elem, HB, NW, MODE == kDirect>(a, st, lds, &arrivals, qh0, out_row, d, lane, wave))
      return;
    if constexpr (fused) arrive<Elem>(a, u, qh0, lane, 0, 1, fused_all);
  } else {
    combine_waves<Elem, HB, NW, MODE == kDirect>(a, st, lds, qh0, out_row, d, tid, lane, wave);
    if constexpr (fused) arrive<Elem>(a, u, qh0, lane, wave, kWaves, fused_all);
  }
}

// ---------------------------------------------------------------------------------
// Segmented LSE merge kernel: one wave per (row, query head).  Grid-split slots are
// ((row*Hq + qh)*S + s) (cuh:719-751); work-queue slots are (split_offsets[row] + s)*Hq
// + qh (cuh:753-784).
// ---------------------------------------------------------------------------------
struct MergeArgs {
  const float* part_m;
  const float* part_l;
  const float* part_acc;
  const int32_t* seq_lens;       // queue mode
  const int32_t* split_offsets;  // queue mode
  const int32_t* out_indices;
  uint8_t* out;
  int32_t batch, hq, out_rows;
  int32_t num_splits;            // split mode
  int32_t total_slots;           // queue mode
  int32_t context, max_tokens;   // split mode length fallback / clamp
  int32_t num_tasks, hkv;        // queue mode: the queue's item count (-1: unknown) and Hkv
};

template <class Elem, bool QUEUE>
__global__ __launch_bounds__(64) void merge_kernel(MergeArgs a) {
  const int wave_id = blockIdx.x;  // one wave per workgroup
  const int lane = threadIdx.x;
  if (wave_id >= a.batch * a.hq) return;
  const int row = uniform(wave_id / a.hq);
  const int qh = uniform(wave_id - row * a.hq);
  // The output row is loaded first and waited for last, so it costs no round trip of its own.
  const int out_row_loaded = load_vector_deferred(a.out_indices ? a.out_indices + row : nullptr);
  int count, total = 0, nsplit = 1, split0 = 0;
  bool all = false;  // queue mode: every slot of the row is folded
  long base, stride;
  SlotChunk guessed;
  bool hit = false;
  if (QUEUE) {
    // With a fixed split count every row owns total_slots / batch slots.  The first chunk
    // of that slot range is loaded right behind the row's offsets and length and used when
    // the offsets match: the merge then waits for one memory round trip instead of two.
    // (Vector loads complete in issue order, so the offsets can be waited for alone.)
    const int so_first = load_vector_deferred(a.split_offsets);
    const int so_last = load_vector_deferred(a.split_offsets + a.batch);
    const int o0 = load_vector_uniform(a.split_offsets + row);
    const int o1 = load_vector_uniform(a.split_offsets + row + 1);
    int len = load_vector_uniform(a.seq_lens + row);
    all = a.num_tasks >= 0 && queue_writes_every_slot(a.num_tasks, a.hkv, uniform(so_first),
                                                      uniform(so_last));
    const int per_row = a.total_slots / a.batch;
    const bool guess = per_row > 0 && per_row * a.batch == a.total_slots;
    load_chunk_if(guessed, a.part_m, a.part_l, a.part_acc, (long)row * per_row * a.hq + qh, a.hq,
                  per_row < 1 ? 1 : (per_row < kMergeChunk ? per_row : kMergeChunk), lane, guess);
    hit = guess && o0 == row * per_row && o1 - o0 == per_row;
    const int first = o0 < 0 ? 0 : o0;
    const int last = o1 > a.total_slots ? a.total_slots : o1;
    count = last - first;
    nsplit = o1 - o0;
    split0 = first - o0;
    if (len > a.max_tokens) len = a.max_tokens;
    total = ceil_tiles(len < 0 ? 0 : len);
    base = (long)first * a.hq + qh;
    stride = a.hq;
  } else {
    count = a.num_splits;
    base = ((long)row * a.hq + qh) * a.num_splits;
    stride = 1;
  }
  // In split mode the slot range needs no memory read: the merge costs one memory round
  // trip (the states), as it does in queue mode when the fixed-split guess holds.
  LseAcc acc;
  int c_begin = 0;
  if (QUEUE) {
    // Chunk 0: the guessed loads when the offsets matched, else loaded now (a descriptor
    // that covers nothing when the row has no slots).  The guessed values are selected,
    // not branched on, so their loads stay ahead of the wait for the offsets.
    const int n = count < 1 ? 1 : (count < kMergeChunk ? count : kMergeChunk);
    SlotChunk c;
    if (!hit) load_chunk_if(c, a.part_m, a.part_l, a.part_acc, base, stride, n, lane, count > 0);
    c.ms = hit ? guessed.ms : c.ms;
    c.ls = hit ? guessed.ls : c.ls;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) c.v[j] = hit ? guessed.v[j] : c.v[j];
    acc.fold(lane < count && lane < kMergeChunk &&
                 slot_live<QUEUE>(lane, count, total, nsplit, split0, all),
             c.ms, c.ls, c.v);
    c_begin = kMergeChunk;
  }
  fold_slots<QUEUE, false>(acc, a.part_m, a.part_l, a.part_acc, base, stride, count, total, nsplit,
                           split0, lane, c_begin, all);
  const int out_row = a.out_indices ? uniform(out_row_loaded) : row;
  if (out_row < 0 || out_row >= a.out_rows) return;
  acc.store<Elem>(a.out + ((long)out_row * a.hq + qh) * kD * 2, lane);
}

// ---------------------------------------------------------------------------------
// Balanced work-queue schedule.  A complete work queue (every non-empty split of every
// (row, kv head) pair, as the builder emits it) covers each pair's tiles
// [0, ceil(len / 32)) once, whatever its split counts; the combined work-queue op can
// therefore stream those tiles with an equal share per wave instead of one workgroup per
// item.  Each (row, kv head) pair with tiles is laid out as kBalPieceCost start-up
// positions followed by its tiles, pairs end to end (rows in order, kv heads within a
// row), T positions in all; wave v of V takes positions [floor(v T / V), floor((v + 1) T
// / V)), cutting pairs anywhere, and writes one partial state per pair piece that holds
// tiles.  The start-up positions carry no work: they charge each piece its fixed cost
// (the Q loads, the first page lookups and the pipeline ramp, ~1-1.5 us per piece against
// ~0.5-0.8 us per tile per wave in per-wave timestamps), so a wave that starts many short
// rows takes fewer tiles.  The piece of pair p in wave v goes to state group p + v: pieces
// are intervals of both orderings, so no two pieces share a group, and the pieces of one
// pair lie in the groups p + va .. p + vb, va and vb the waves of its first and last tile
// (position x is in wave ceil((x + 1) V / T) - 1).  When T < V some waves hold no
// position; their groups are skipped by the same rule as the empty splits of a work
// queue.  A group holds the pair's G query heads; there are at most B * Hkv + V - 1
// groups.  Waves run at most one per SIMD with two tiles in flight, with no LDS and no
// barrier: two per CU for 2-byte K/V, four for fp8 (bal_waves_per_cu); the merge reads
// the layout from the plan entries.  The per-item schedule ends
// with a tail: C4 steps put 1.25 long items on some CUs and 2 on others, and the CUs with
// two finish ~8 us later (per-wave timestamps of the decode kernel).
// ---------------------------------------------------------------------------------
// Waves per workgroup and per CU.  With 2-byte K/V two waves (one tile computed and
// one in flight each, 64 KB per CU) stream as fast as four and cut the pieces and merge
// states in half: C4 decode 36.7-37.0 against 37.0-37.2 us, C5 G=8 196.5-197.1 against
// 197.9-198.4 us (one wave: 42.7 and 236-237 us).  An fp8 tile carries half the bytes and
// the same compute, and needs all four SIMDs: 21.9 us with four waves, 25.6-25.8 with two.
constexpr int kBalWavesMax = 4;
constexpr int bal_waves_per_cu(bool fp8) { return fp8 ? 4 : 2; }
constexpr int kBalRowChunks = 4;  // lane l holds rows l + 64k, k < 4: batches up to 256
constexpr int kBalPieceCost = 2;  // start-up positions of each (row, kv head) pair

// The rows of a launch as one wave holds them: lane l keeps rows l + 64k (chunk k).  A
// row weighs (kBalPieceCost + tiles) * Hkv positions, 0 without tiles; incl is the
// inclusive prefix of weights in row order
// (rows past the batch weigh 0, so their prefix is the total).  The four chunks are
// separate registers, never an array, so that selecting one by a run-time chunk index
// does not put the table in scratch memory.
struct RowTable {
  int len0, len1, len2, len3;
  long incl0, incl1, incl2, incl3;
  long total;
};

// One DPP step of the scan: x plus the value of the lane `ctrl` selects (0 where it selects
// none, or in the rows row_mask leaves out), on both 32-bit halves.
template <int CTRL, int ROW_MASK>
__device__ inline long dpp_add(long x) {
  const uint64_t u = (uint64_t)x;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf, false);
  return x + (long)(((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum over the wave's 64 lanes with DPP (no LDS): within each row of 16
// lanes by shifts of 1, 2, 4 and 8, then row 0's total into rows 1 and 3 (row_bcast:15)
// and rows 0-1's into rows 2 and 3 (row_bcast:31).
__device__ inline long wave_incl_scan(long x, int) {
  x = dpp_add<0x111, 0xf>(x);  // row_shr:1
  x = dpp_add<0x112, 0xf>(x);  // row_shr:2
  x = dpp_add<0x114, 0xf>(x);  // row_shr:4
  x = dpp_add<0x118, 0xf>(x);  // row_shr:8
  x = dpp_add<0x142, 0xa>(x);  // row_bcast:15
  x = dpp_add<0x143, 0xc>(x);  // row_bcast:31
  return x;
}

__device__ inline long read_lane64(long x, int src) {
  const uint64_t u = (uint64_t)x;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, src);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), src);
  return (long)(((uint64_t)hi << 32) | lo);
}

// One chunk: the clamped length of row lane + 64k and its inclusive prefix (carry in/out).
__device__ inline void row_chunk(const DecodeArgs& a, int lane, int k, int raw, int& len,
                                 long& incl, long& carry) {
  const int r = lane + 64 * k;
  len = r < a.batch ? clamp_length(a, raw) : 0;
  const int tiles = ceil_tiles(len);
  incl = wave_incl_scan(tiles > 0 ? (long)(tiles + kBalPieceCost) * a.hkv : 0, lane) + carry;
  carry = read_lane64(incl, 63);
}

// Loads every row's length and builds the prefix of row weights.  batch <= 64 *
// kBalRowChunks (checked on the host).  The lengths are read through one buffer descriptor
// that covers seq_lens[0, batch): the four loads go out together with no branch between
// them, and lanes past the batch read 0 without touching memory.
// Lanes' raw values of an int32 array at rows lane + 64k, k < 4, read through one buffer
// descriptor over [0, n): the four loads go out together, and lanes past n read 0.
struct RowInts {
  int v0, v1, v2, v3;
};
__device__ inline RowInts load_row_ints(const int32_t* p, int n, int lane, int shift = 0) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(p), (short)0, uniform(n > 0 ? n * 4 : 0), kRsrcWord3);
  const int o = 4 * (lane + shift);
  return RowInts{(int)__builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0),
                 (int)__builtin_amdgcn_raw_buffer_load_b32(r, o + 256, 0, 0),
                 (int)__builtin_amdgcn_raw_buffer_load_b32(r, o + 512, 0, 0),
                 (int)__builtin_amdgcn_raw_buffer_load_b32(r, o + 768, 0, 0)};
}

__device__ inline void row_table_from(const DecodeArgs& a, int lane, const RowInts& raw,
                                      RowTable& t) {
  const int raw0 = raw.v0, raw1 = raw.v1, raw2 = raw.v2, raw3 = raw.v3;
  // Chunks past the batch hold no row: their prefix is the total.
  long carry = 0;
  row_chunk(a, lane, 0, raw0, t.len0, t.incl0, carry);
  t.len1 = t.len2 = t.len3 = 0;
  if (a.batch > 64) row_chunk(a, lane, 1, raw1, t.len1, t.incl1, carry);
  if (a.batch > 128) row_chunk(a, lane, 2, raw2, t.len2, t.incl2, carry);
  if (a.batch > 192) row_chunk(a, lane, 3, raw3, t.len3, t.incl3, carry);
  if (a.batch <= 64) t.incl1 = carry;
  if (a.batch <= 128) t.incl2 = carry;
  if (a.batch <= 192) t.incl3 = carry;
  t.total = carry;
}

__device__ inline void row_table(const DecodeArgs& a, int lane, RowTable& t) {
  row_table_from(a, lane, load_row_ints(a.seq_lens, a.batch, lane), t);
}

// Length and inclusive prefix of row r (wave-uniform r): each chunk's value at lane r % 64
// is read, then the chunk r / 64 is selected.
__device__ inline int table_len(const RowTable& t, int r) {
  const int k = r >> 6, l = r & 63;
  const int v0 = __builtin_amdgcn_readlane(t.len0, l), v1 = __builtin_amdgcn_readlane(t.len1, l);
  const int v2 = __builtin_amdgcn_readlane(t.len2, l), v3 = __builtin_amdgcn_readlane(t.len3, l);
  return k == 0 ? v0 : (k == 1 ? v1 : (k == 2 ? v2 : v3));
}
__device__ inline long table_incl(const RowTable& t, int r) {
  const int k = r >> 6, l = r & 63;
  const long v0 = read_lane64(t.incl0, l), v1 = read_lane64(t.incl1, l);
  const long v2 = read_lane64(t.incl2, l), v3 = read_lane64(t.incl3, l);
  return k == 0 ? v0 : (k == 1 ? v1 : (k == 2 ? v2 : v3));
}

// Row holding position x (0 <= x < total): the number of rows whose prefix is at most x.
__device__ inline int table_row(const RowTable& t, long x) {
  return __builtin_popcountll(__builtin_amdgcn_ballot_w64(t.incl0 <= x)) +
         __builtin_popcountll(__builtin_amdgcn_ballot_w64(t.incl1 <= x)) +
         __builtin_popcountll(__builtin_amdgcn_ballot_w64(t.incl2 <= x)) +
         __builtin_popcountll(__builtin_amdgcn_ballot_w64(t.incl3 <= x));
}

// ---------------------------------------------------------------------------------
// Queue check of the balanced schedule.  The schedule streams each (row, kv head) pair's
// tiles [0, T) once, which is what the reference computes for the queue that
// compile_persistentkv_metadata builds (benchmark_serving_trace.py:668-729): for each row
// in order, each split s of its S = split_offsets[row + 1] - split_offsets[row] with a
// non-empty row-local range [T s / S, T (s + 1) / S) (cuh:330-337), the items
// (row, kvh, s, range) for kvh = 0 .. Hkv - 1.  The queue is that one when
// - every row has S >= 0, and S >= 1 when it has tiles; split_offsets[0] >= 0 and
//   split_offsets[B] <= total_slots;
// - num_tasks = Hkv x sum over rows of min(S, T) (the non-empty splits);
// - every item idx = (r, k, s, tb, te) has 0 <= r < B, 0 <= k < Hkv, 0 <= s < S_r, the
//   row-local range of split s (a negative bound standing for it, cuh:330-337), which is
//   non-empty, and idx = Hkv x (P_r + n) + k, with P_r the non-empty splits of the rows
//   before r and n = min(s, tb) those of row r before split s (with T >= S every split
//   is non-empty, n = s; with T < S each holds one tile, n = tb).
// The index rule maps distinct (r, s, k) to distinct positions of [0, num_tasks), so such
// a queue holds each expected item once and nothing else.  Decode workgroup w checks the
// row conditions and the items [w c, (w + 1) c), c = ceil(num_tasks / workgroups), in its
// wave 0 before that wave's pieces (~5 items at C4's 1,280 over 256 workgroups; checking
// every item in every workgroup cost the decode ~3 us, checking after the pieces ~0.7 us,
// against ~0.3 us here), and writes the result to bal_flags[w]; the merge reads every
// flag, and on any failure computes the pairs itself (balanced_merge_fallback).
// ---------------------------------------------------------------------------------
constexpr int kRowEntry = 4;                                   // ints per row: {P, T, S, len}

// Fields of up to 64 items, one per lane: items first + lane (buffer loads that read 0 past
// num_tasks).
struct ItemLane {
  int f[5];
};
__device__ inline ItemLane load_item_lane(const DecodeArgs& a, long first, int lane) {
  const long idx = first + lane;
  const int off = idx < a.num_tasks ? (int)(idx * 20) : 0;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(a.work_items), (short)0, uniform(a.num_tasks * 20), kRsrcWord3);
  ItemLane it;
#pragma unroll
  for (int q = 0; q < 5; ++q)
    it.f[q] = idx < a.num_tasks ? (int)__builtin_amdgcn_raw_buffer_load_b32(r, off + 4 * q, 0, 0) : 0;
  return it;
}

// Whether item idx (fields f) is the builder's idx-th item; e is the row entry of row f[0]
// clamped into the batch.
__device__ inline bool item_is_builders(const DecodeArgs& a, long idx, const int (&f)[5],
                                        const i32x4& e) {
  const int r = f[0], k = f[1], s = f[2];
  const long T = e[1], S = e[2];
  const bool fields = (unsigned)r < (unsigned)a.batch && (unsigned)k < (unsigned)a.hkv &&
                      s >= 0 && s < S;
  const long ts = T * s, ts1 = ts + T;
  long tb = f[3], te = f[4];
  // A negative bound stands for the row-local one (a division, taken only when a lane of
  // the wave has such a bound; the builder writes none).
  if (__builtin_amdgcn_ballot_w64(fields && (tb < 0 || te < 0)) != 0) {
    const long Sd = S > 0 ? S : 1;
    if (tb < 0) tb = ts / Sd;
    if (te < 0) te = ts1 / Sd;
  }
  // tb = floor(T s / S) and te = floor(T (s + 1) / S), checked without dividing.
  const bool bounds = tb * S <= ts && ts < (tb + 1) * S && te * S <= ts1 && ts1 < (te + 1) * S;
  const long n = T >= S ? s : tb;
  return idx >= a.num_tasks ||
         (fields && bounds && te > tb && idx == (long)a.hkv * (e[0] + n) + k);
}

// One chunk of the row table for the check: lane holds row r = lane + 64 k; returns its
// count of non-empty splits and folds the row-level conditions into ok.
__device__ inline long check_row(const DecodeArgs& a, int lane, int k, int len, int so0, int so1,
                                 bool& ok) {
  const int r = lane + 64 * k;
  if (r >= a.batch) return 0;
  const int T = ceil_tiles(len);
  const int S = so1 - so0;
  if (S < 0 || (T > 0 && S < 1)) ok = false;
  return T > 0 && S > 0 ? (S < T ? S : T) : 0;
}

// This workgroup's part of the check, by one wave: the row conditions, then the items
// [first, first + count) against a table of the rows {P, T, S, len} in the wave's LDS
// `rows` (a wave's LDS stores are visible to its later LDS loads).  `lead` holds items
// first .. first + 63 as loaded at the kernel's start.
__device__ inline bool check_queue_part(const DecodeArgs& a, const RowTable& t, const RowInts& so0,
                                        const RowInts& so1, int so_last, int32_t* rows,
                                        const ItemLane& lead, long first, long count, int lane) {
  bool ok = true;
  const int lens[4] = {t.len0, t.len1, t.len2, t.len3};
  const int s0[4] = {so0.v0, so0.v1, so0.v2, so0.v3};
  const int s1[4] = {so1.v0, so1.v1, so1.v2, so1.v3};
  long carry = 0;
#pragma unroll
  for (int k = 0; k < kBalRowChunks; ++k) {
    if (k * 64 >= a.batch) break;
    const long ne = check_row(a, lane, k, lens[k], s0[k], s1[k], ok);
    const long incl = wave_incl_scan(ne, lane) + carry;
    carry = read_lane64(incl, 63);
    const int r = lane + 64 * k;
    if (r < a.batch) {
      const long p = incl - ne;
      *(i32x4*)(rows + r * kRowEntry) =
          i32x4{p < 0x7fffffffL ? (int)p : 0x7fffffff, ceil_tiles(lens[k]), s1[k] - s0[k], lens[k]};
    }
  }
  ok = __builtin_amdgcn_ballot_w64(!ok) == 0;
  ok = ok && a.num_tasks == (long)a.hkv * carry && uniform(s0[0]) >= 0 && so_last <= a.total_slots;
  for (long c0 = 0; c0 < count; c0 += 64) {
    const ItemLane it = c0 == 0 ? lead : load_item_lane(a, first + c0, lane);
    const int r = (unsigned)it.f[0] < (unsigned)a.batch ? it.f[0] : 0;
    const i32x4 e = *(const i32x4*)(rows + r * kRowEntry);
    const bool mine = c0 + lane < count;
    ok = ok && __builtin_amdgcn_ballot_w64(mine && !item_is_builders(a, first + c0 + lane, it.f, e)) == 0;
  }
  return ok;
}

// One workgroup of bal_waves_per_cu independent waves per CU (the launch asks for enough
// LDS that no two share a CU).
template <class Elem, int PG>
__global__ __launch_bounds__(bal_waves_per_cu(PG == kPgFp8) * 64) __attribute__((amdgpu_waves_per_eu(1)))
void balanced_decode_kernel(DecodeArgs a) {
  constexpr int kWaves = bal_waves_per_cu(PG == kPgFp8);
  extern __shared__ int32_t bal_lds[];  // wave 0: the row table of the queue check
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const long V = (long)gridDim.x * kWaves;
  const long v = (long)blockIdx.x * kWaves + wave;
  // This workgroup's items of the queue check (wave 0), loaded with the lengths and slot
  // offsets; lanes past the queue load nothing.
  const int per_wg = (int)(((unsigned)a.num_tasks + gridDim.x - 1) / gridDim.x);
  const long item0 = (long)blockIdx.x * per_wg;
  const long items = item0 >= a.num_tasks ? 0 : (a.num_tasks - item0 < per_wg ? a.num_tasks - item0 : per_wg);
  RowTable t;
  if (wave == 0) {
    const RowInts lens = load_row_ints(a.seq_lens, a.batch, lane);
    const RowInts so0 = load_row_ints(a.split_offsets, a.batch + 1, lane);
    const RowInts so1 = load_row_ints(a.split_offsets, a.batch + 1, lane, 1);
    const int so_last = load_vector_deferred(a.split_offsets + a.batch);
    const ItemLane lead = load_item_lane(a, items > 0 ? item0 : a.num_tasks, lane);
    row_table_from(a, lane, lens, t);
    const bool ok = check_queue_part(a, t, so0, so1, uniform(so_last), bal_lds, lead, item0, items, lane);
    if (lane == 0) a.bal_flags[blockIdx.x] = ok ? 1 : 0;
  } else {
    row_table(a, lane, t);
  }
  const long T = t.total;
  long x = v * T / V;
  const long x1 = (v + 1) * T / V;
  const int G = a.group;
  while (x < x1) {
    const int r = uniform(table_row(t, x));  // a row with tiles: others hold no position
    const int len = uniform(table_len(t, r));
    const int tiles = ceil_tiles(len);
    const long span = tiles + kBalPieceCost;  // positions of each of the row's pairs
    const long off = x - (table_incl(t, r) - span * a.hkv);
    const int kvh = uniform((int)(off / span));
    const long pair0 = x - off + kvh * span;  // first position of pair (r, kvh)
    const long e = x - pair0;                 // 0 <= e < span
    const int t0 = uniform((int)(e > kBalPieceCost ? e - kBalPieceCost : 0));
    const long lim = x1 - pair0 - kBalPieceCost;  // tiles of the pair within this wave
    const int t1 = uniform(lim < tiles ? (int)(lim > 0 ? lim : 0) : tiles);
    if (t1 <= t0) break;  // the range ends among the pair's start-up positions
    // The query row is requested first and waited for only at the Q loads; the first two
    // block-table reads go out beside it.
    const int q_loaded = load_vector_lanes(a.q_indices ? a.q_indices + r : nullptr,
                                           a.batch < 0 ? lane : 0);  // batch > 0 here
    FastPager::Pages f0, f1;
    {
      const FastPager pg(a, r, kvh, 0, lane);
      f0 = pg.lookup(t0);
      f1 = pg.lookup(t0 + 1);
    }
    const int qh0 = kvh * G;
    u32x4 qf[1][4];
    load_q<1, PG == kPgFp8>(a, q_loaded, r, qh0, lane, qf);
    if (t0 == 0) {
      // The wave that holds the pair's first tile records the waves its tiles span (the
      // last tile, pair0 + kBalPieceCost + tiles - 1, lies in wave ceil((x + 1) V / T) - 1)
      // while its first loads are in flight: the merge then needs no row table.
      const long vb = ((pair0 + kBalPieceCost + tiles) * V + T - 1) / T - 1;
      if (lane == 0)
        *(u32x4*)(a.bal_plan + ((long)r * a.hkv + kvh) * 4) =
            u32x4{(uint32_t)v, (uint32_t)(vb - v + 1), (uint32_t)T, (uint32_t)(T >> 32)};
    }
    WaveState<1> st;
    init_state<1>(st);
    stream_unit<Elem, 1, PG, 2>(a, st, qf, r, kvh, t0, t1, len, lane, true, f0, f1);
    const long group = (long)r * a.hkv + kvh + v;
    const Dest d{a.part_m, a.part_l, a.part_acc, group * G, 1, false};
    write_wave_state<Elem, 1, false>(a, st, qh0, 0, d, lane);
    x = pair0 + kBalPieceCost + t1;
  }

}

// The merge's answer for a queue other than the builder's (some decode workgroup's check
// failed), for the G query heads of pair (row, kvh), by one wave.  The reference's result
// for such a queue (each slot of the row folded, a slot holding the state of the item that
// writes it) is attention over the union of the row's items' tile ranges, with unwritten
// slots taken as neutral as the per-item schedule takes the builder's empty splits.  The
// wave scans the whole queue and streams the ranges of the pair's valid items (row and kv
// head the pair's, split below the row's slot count, slot inside the workspace) in queue
// order into one state, and writes the normalised output.  Slow (a pass over the queue
// and a serial stream per pair), and only for queues other than the builder's; the fused
// append's token is already in the pool (the decode wrote it).
template <class Elem, int PG>
__device__ void balanced_merge_fallback(const DecodeArgs& a, int row, int kvh, int out_row, int lane) {
  const int len = uniform(clamp_length(a, a.seq_lens[row]));
  const int T = ceil_tiles(len);
  const int so0 = uniform(a.split_offsets[row]);
  const int S = uniform(a.split_offsets[row + 1]) - so0;
  const int G = a.group;
  const int q_loaded = a.q_indices ? a.q_indices[row] : 0;
  u32x4 qf[1][4];
  load_q<1, PG == kPgFp8>(a, q_loaded, row, kvh * G, lane, qf);
  WaveState<1> st;
  init_state<1>(st);
  for (long i0 = 0; T > 0 && i0 < a.num_tasks; i0 += 64) {
    const ItemLane it = load_item_lane(a, i0, lane);
    const int s = it.f[2];
    const bool match = i0 + lane < a.num_tasks && it.f[0] == row && it.f[1] == kvh && s >= 0 &&
                       s < S && (long)so0 + s >= 0 && (long)so0 + s < a.total_slots;
    uint64_t hits = __builtin_amdgcn_ballot_w64(match);
    while (hits) {
      const int src = __builtin_ctzll(hits);
      hits &= hits - 1;
      const int ss = __builtin_amdgcn_readlane(s, src);
      long tb = __builtin_amdgcn_readlane(it.f[3], src), te = __builtin_amdgcn_readlane(it.f[4], src);
      if (tb < 0) tb = (long)T * ss / S;
      if (te < 0) te = (long)T * (ss + 1) / S;
      const int t0 = uniform((int)(tb < 0 ? 0 : tb)), t1 = uniform((int)(te > T ? T : te));
      if (t1 > t0) stream_tiles<Elem, 1, PG, 2>(a, st, qf, row, kvh, t0, t1, len, lane);
    }
  }
  finish_state<1>(st);
  const Dest d{nullptr, nullptr, nullptr, 0, 1, false};
  write_wave_state<Elem, 1, true>(a, st, kvh * G, out_row, d, lane);
}

// Whether every decode workgroup's part of the queue check passed (bal_flags[0, n)), by
// one wave: 16-byte loads, all issued together for up to 1024 workgroups.
__device__ inline bool queue_checks_passed(const DecodeArgs& a, int n, int lane) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(a.bal_flags), (short)0, uniform(n * 4), kRsrcWord3);
  bool ok = true;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k * 256 >= n) break;
    const u32x4 f = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (k * 64 + lane) * 16, 0, 0));
#pragma unroll
    for (int q = 0; q < 4; ++q) ok = ok && (k * 256 + lane * 4 + q >= n || f[q] == 1);
  }
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// Merge of the balanced schedule: one workgroup of nw = blockDim.x / 64 waves (1, 2 or
// kBalMergeWaves: at most the decode's waves per CU) per (row, query head) folds the
// groups of its pair (the decode's waves va .. va + count - 1 of `waves`, from the pair's
// plan entry): wave w folds the w-th of nw equal shares of the groups, and the partial
// merges are combined through LDS.  A few long pairs (~35 groups each at 8 rows with two
// decode waves per CU) take 2 waves each; many short rows take one wave each, so that the
// whole grid is resident at once (the kernel needs ~165 VGPRs, ~250 with the wide fold).
constexpr int kBalMergeWaves = 4;

template <class Elem, bool WIDE, int PG>
__global__ __launch_bounds__(kBalMergeWaves * 64) void balanced_merge_kernel(DecodeArgs a, int waves,
                                                                             int check_wgs) {
  __shared__ float sm_ml[kBalMergeWaves][2];
  __shared__ f32x2 sm_a[kBalMergeWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int nw = uniform(blockDim.x >> 6);
  const int wg = blockIdx.x;
  if (wg >= a.batch * a.hq) return;  // whole workgroup
  const int row = uniform(wg / a.hq);
  const int qh = uniform(wg - row * a.hq);
  const int kvh = uniform(qh / a.group), h = qh - kvh * a.group;
  // One round trip: the output row, the row's length and the pair's plan entry (written by
  // the decode's wave that holds the pair's first tile) are loaded together.
  const int out_row_loaded = load_vector_deferred(a.out_indices ? a.out_indices + row : nullptr);
  const int len_loaded = load_vector_deferred(a.seq_lens + row);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(a.bal_plan + ((long)row * a.hkv + kvh) * 4), (short)0, a.bal_plan ? 16 : 0,
      kRsrcWord3);  // a null plan reads zeros
  const u32x4 plan = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, 0, 0, 0));
  // The decode's queue check, in the same round trip.  A queue other than the builder's is
  // computed here instead, pair by pair, by the first query head's workgroup.
  if (!queue_checks_passed(a, check_wgs, lane)) {
    if (h == 0 && wave == 0) {
      const int out_row = a.out_indices ? uniform(out_row_loaded) : row;
      balanced_merge_fallback<Elem, PG>(a, row, kvh, out_row, lane);
    }
    return;
  }
  // Selected, not branched on, so that the plan load is issued beside the length load.
  // Clamped so that the state loads stay inside the workspace whatever it holds.
  int va = uniform((int)plan[0]);
  va = va < 0 ? 0 : (va >= waves ? waves - 1 : va);
  int count = uniform((int)plan[1]);
  count = count < 0 ? 0 : (count > waves - va ? waves - va : count);
  const long T = (long)(((uint64_t)(uint32_t)uniform((int)plan[3]) << 32) | (uint32_t)uniform((int)plan[2]));
  if (ceil_tiles(clamp_length(a, uniform(len_loaded))) == 0) count = 0;  // no plan entry
  const long base = ((long)row * a.hkv + kvh + va) * a.group + h;
  // This wave's share of the groups [c0, c1).
  const int c0 = count * wave / nw, c1 = count * (wave + 1) / nw;
  LseAcc acc;
  // Groups of waves with no position are skipped, as the empty splits of a queue are.  A
  // share of more than one chunk is folded in one round trip when it fits.
  if (WIDE && c1 - c0 > kMergeChunk && c1 - c0 <= kWideStates)
    fold_wide(acc, a.part_m, a.part_l, a.part_acc, base + (long)c0 * a.group, a.group, c1 - c0, T,
              waves, va + c0, lane);
  else
    fold_slots_pipelined<true>(acc, a.part_m, a.part_l, a.part_acc, base + (long)c0 * a.group,
                               a.group, c1 - c0, T, waves, va + c0, lane);
  float M = acc.M, L = acc.L;
  f32x2 A = acc.A;
  if (nw > 1) {
    if (lane == 0) {
      sm_ml[wave][0] = acc.M;
      sm_ml[wave][1] = acc.L;
    }
    sm_a[wave][lane] = acc.A;
    __syncthreads();
    if (wave != 0) return;
    M = -FLT_MAX;
    for (int w = 0; w < nw; ++w) M = fmaxf(M, sm_ml[w][0]);
    L = 0.f;
    A = f32x2{0.f, 0.f};
    for (int w = 0; w < nw; ++w) {
      const float e = __builtin_amdgcn_exp2f((sm_ml[w][0] - M) * kLog2e);
      L += e * sm_ml[w][1];
      A += e * sm_a[w][lane];
    }
  }
  const int out_row = a.out_indices ? uniform(out_row_loaded) : row;
  if (out_row < 0 || out_row >= a.out_rows) return;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  *(uint32_t*)(a.out + ((long)out_row * a.hq + qh) * kD * 2 + 4 * lane) =
      Elem::pack2(A[0] * inv, A[1] * inv);
}

// ---------------------------------------------------------------------------------
// Host side: validation, dispatch and launch.
// ---------------------------------------------------------------------------------
thread_local char g_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_error[0] = '\0';
  return PKV_OK;
}

int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int s = 0;
  while ((1 << s) < x) ++s;
  return s;
}

// LDS of a decode workgroup: the barrier combine stages O in chunks of heads (8 with 8
// waves, 16 with 4); the barrier-free combine holds every wave's O at once.
size_t lds_bytes(int G, int nw, bool async = false) {
  const int chunk = async ? G : (nw == 8 ? 8 : 16);
  return (size_t)(3 * nw * 32 + nw * (G < chunk ? G : chunk) * kD) * sizeof(float);
}

struct Geometry {
  int batch, hq, hkv, head_dim, num_pages, page_size, max_pages, dtype;
};

int check_geometry(const Geometry& g, const void* q, const void* k, const void* v,
                   const void* table, const void* out) {
  if (g.head_dim != kD)
    return fail(PKV_ERR_UNSUPPORTED, "PersistentKV extension currently requires d=128");
  if (g.dtype != PKV_DTYPE_F16 && g.dtype != PKV_DTYPE_BF16)
    return fail(PKV_ERR_UNSUPPORTED, "dtype must be fp16 or bf16");
  if (g.hkv <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "Hkv must be positive");
  if (g.hq % g.hkv != 0) return fail(PKV_ERR_INVALID_ARGUMENT, "Hq must be divisible by Hkv");
  const int G = g.hq / g.hkv;
  if (G < 1 || G > PKV_MAX_GROUP)
    return fail(PKV_ERR_UNSUPPORTED, "PersistentKV supports G=Hq/Hkv in [1,32]; got G=%d from Hq=%d Hkv=%d",
                G, g.hq, g.hkv);
  if (g.page_size <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "page_size must be positive");
  if (g.batch < 0) return fail(PKV_ERR_INVALID_ARGUMENT, "batch must be non-negative");
  if (g.num_pages <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "k_pages must hold at least one page");
  if (g.max_pages <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "block_table must have at least one column");
  if (g.batch > 0 && (!q || !k || !v || !table || !out))
    return fail(PKV_ERR_INVALID_ARGUMENT, "a required pointer is null");
  if ((long)g.hkv * g.page_size * kD * 2 > 0x7fffffffL)
    return fail(PKV_ERR_UNSUPPORTED, "page too large (Hkv*page_size*256 must fit in 31 bits)");
  return PKV_OK;
}

// Waves per decode workgroup.  With every CU streaming, 32-64 KB in flight per CU already
// holds HBM at its ceiling, and a launch ends about one loaded latency after its last
// requests, a latency that grows with the bytes in flight (probes: 1.3 us at 32 KB per CU,
// 5.4 us at 128 KB, the same bandwidth).  So the grid ops (direct and split units) keep
// little in flight:
//   - at most one unit per CU: 2 waves with two 16 KB tiles in flight each, one workgroup
//     per CU (C3 at 32k 27.15 against 27.5 us with 4 x 1, B1 G4 32k 26.7 against 28.1 us,
//     C3 at 16k 17.6 against 18.3 us);
//   - more units: 4 waves with one tile each (C2, 8 units per CU: 106.3 us, against 107.9
//     with 8 waves and 110.5 with 2 x 2).
// Work-queue items (the per-item schedule) keep eight, which spread a long item over more
// waves (per-item C4: 52.2 against 55.4 us with 4).  G > 16 runs one wave per SIMD with
// two tiles in flight and stays at four.  PKV_DECODE_WAVES=2|4|8 overrides the choice.
int cu_count();

int decode_waves(int hb, int mode, int units) {
  static const int forced = [] {
    const char* e = getenv("PKV_DECODE_WAVES");
    return e ? atoi(e) : 0;
  }();
  if (hb > 1) return 4;
  if (forced == 2 || forced == 4 || forced == 8) return forced;
  if (mode == kQueue) return 8;
  return units <= cu_count() ? 2 : 4;
}

// Compute units of the current device (cached per device).
int cu_count() {
  static int cache[64] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  if (cache[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0)
      n = 256;
    cache[device] = n;
  }
  return cache[device];
}

// The barrier-free combine for launches of at least 3 units per CU (measured: C4 with 4.3
// units per CU and C2 with 8 gain 2 %; C3 with 1 and C5 G=8 with 2.2 lose 2 %, since
// one wave combining alone lengthens a unit's critical path).  PKV_ASYNC_COMBINE=0|1
// forces the choice (tuning).
bool use_async_combine(int units) {
  static const int forced = [] {
    const char* e = getenv("PKV_ASYNC_COMBINE");
    return e ? (e[0] == '0' ? 0 : 1) : -1;
  }();
  if (forced >= 0) return forced == 1;
  return units >= 3 * cu_count();
}

// A work-queue launch with the fused merge (merge_counters set) runs its own kernel: the
// arrivals and the in-kernel merge are compiled only into it, so the unfused kernel's
// tile loop keeps the scalar registers they would take (the queue kernels spilled
// 350-395 SGPRs with both paths in one kernel).
template <class Elem, int HB, int PG, int MODE, int NW, bool ASYNC, int DEPTH = HB>
void launch_kernel(const DecodeArgs& a, int grid, size_t lds, hipStream_t stream) {
  if constexpr (MODE == kQueue) {
    if (a.merge_counters) {
      decode_kernel<Elem, HB, PG, MODE, NW, ASYNC, DEPTH, true>
          <<<dim3(grid), dim3(NW * 64), lds, stream>>>(a);
      return;
    }
  }
  decode_kernel<Elem, HB, PG, MODE, NW, ASYNC, DEPTH, false><<<dim3(grid), dim3(NW * 64), lds, stream>>>(a);
}

template <class Elem, int HB, int PG, int MODE>
hipError_t launch_decode(const DecodeArgs& a, int grid, hipStream_t stream) {
  const int nw = decode_waves(HB, MODE, grid);
  if constexpr (HB == 1) {
    if (nw == 2) {
      // 96 KB of LDS per workgroup keeps one workgroup, two waves, on each CU.
      launch_kernel<Elem, 1, PG, MODE, 2, false, 2>(a, grid, 96 * 1024, stream);
      return hipGetLastError();
    }
  }
  if (HB == 1 && nw == 8) {
    if constexpr (HB == 1 && PG != kPgGeneric && PG != kPgContig && MODE != kDirect) {
      if (use_async_combine(grid)) {
        launch_kernel<Elem, HB, PG, MODE, 8, true>(a, grid, lds_bytes(a.group, 8, true), stream);
        return hipGetLastError();
      }
    }
    launch_kernel<Elem, HB, PG, MODE, (HB == 1 ? 8 : 4), false>(a, grid, lds_bytes(a.group, 8), stream);
  } else {
    launch_kernel<Elem, HB, PG, MODE, 4, false>(a, grid, lds_bytes(a.group, 4), stream);
  }
  return hipGetLastError();
}

// Direct and split launches of few, long units (at most half the CUs, at least 16 tiles
// each: one row's 8 KV heads with no workspace to split into, or a split launch whose
// workspace holds no sub-splits): each unit is one workgroup on a CU of its own, so the
// launch runs at what one CU streams, and whole-line K loads (Lines) raise that.  8 waves,
// each with two tiles in flight (K in two 8 KB LDS slabs, V in registers: 256 KB per CU,
// 128 KB of LDS, one workgroup per CU).  C1 (8 units of 1 MB): 21.9 us against 30.4 us
// with the K-operand loads; 12 waves with one tile each 22.5 us, 16 waves 25.0 us (128
// registers per wave: the Q fragments spill); 9 or 10 waves with two tiles spill 55-143
// registers.  Units of 8 tiles or fewer are latency-bound and 0.2-0.4 us slower this way
// (the 8-wave combine and the LDS round trip).  PKV_LINES=0|1 forces the choice (tuning,
// tests).
bool use_lines(int mode, int units, int unit_tiles) {
  static const int forced = [] {
    const char* e = getenv("PKV_LINES");
    return e ? (e[0] == '0' ? 0 : 1) : -1;
  }();
  if (mode == kQueue || forced == 0) return false;
  return forced == 1 || (2 * units <= cu_count() && unit_tiles >= 16);
}

constexpr int kLineWaves = 8;

template <class Elem, int PG, int MODE>
hipError_t launch_lines(const DecodeArgs& a, int grid, hipStream_t stream) {
  const size_t lds = std::max<size_t>((size_t)kLineWaves * 2 * kSlabBytes, lds_bytes(a.group, kLineWaves));
  decode_kernel<Elem, 1, PG, MODE, kLineWaves, false, 2>
      <<<dim3(grid), dim3(kLineWaves * 64), lds, stream>>>(a);
  return hipGetLastError();
}

// Contiguous K/V (no block table) runs only the direct and split modes.
template <class Elem, int HB, int MODE>
hipError_t launch_layout(const DecodeArgs& a, int grid, hipStream_t stream) {
  if constexpr (HB == 1 && MODE != kQueue) {
    const int row_tiles = (a.context + kTile - 1) / kTile;
    const int unit_tiles = MODE == kSplit ? row_tiles / a.num_splits : row_tiles;
    if (!a.kv_fp8 && use_lines(MODE, grid, unit_tiles)) {
      if (!a.block_table) return launch_lines<Elem, kPgContigLines, MODE>(a, grid, stream);
      if (a.k_new) return launch_lines<Elem, kPgAppendLines, MODE>(a, grid, stream);  // pages % 16 == 0
      if (a.page_size % 16 == 0) return launch_lines<Elem, kPgLines, MODE>(a, grid, stream);
    }
  }
  if constexpr (MODE != kQueue) {
    if (!a.block_table) return launch_decode<Elem, HB, kPgContig, MODE>(a, grid, stream);
  }
  if (a.kv_fp8) return launch_decode<Elem, HB, kPgFp8, MODE>(a, grid, stream);
  if (a.k_new) return launch_decode<Elem, HB, kPgAppend, MODE>(a, grid, stream);  // pages % 16 == 0
  return (a.page_size % 16) == 0 ? launch_decode<Elem, HB, kPgFast, MODE>(a, grid, stream)
                                 : launch_decode<Elem, HB, kPgGeneric, MODE>(a, grid, stream);
}

template <int MODE>
int dispatch_decode(const DecodeArgs& a, int dtype, int grid, hipStream_t stream) {
  const bool one_block = a.group <= 16;
  hipError_t e;
  if (dtype == PKV_DTYPE_F16)
    e = one_block ? launch_layout<Half, 1, MODE>(a, grid, stream) : launch_layout<Half, 2, MODE>(a, grid, stream);
  else
    e = one_block ? launch_layout<BFloat, 1, MODE>(a, grid, stream)
                  : launch_layout<BFloat, 2, MODE>(a, grid, stream);
  if (e != hipSuccess) return fail(PKV_ERR_LAUNCH, "decode launch failed: %s", hipGetErrorString(e));
  return PKV_OK;
}

// One wave per workgroup, so the (row, head) waves spread over all CUs: each wave's
// ~10 KB of states then shares its CU's load bandwidth with fewer others (measured: C4
// 49.9 against 50.4 us and C1 10.3 against 10.5 us with four waves per workgroup).
int dispatch_merge(const MergeArgs& m, bool queue, int dtype, hipStream_t stream) {
  const int grid = m.batch * m.hq;
  if (grid == 0) return PKV_OK;
  if (dtype == PKV_DTYPE_F16) {
    if (queue) merge_kernel<Half, true><<<grid, 64, 0, stream>>>(m);
    else merge_kernel<Half, false><<<grid, 64, 0, stream>>>(m);
  } else {
    if (queue) merge_kernel<BFloat, true><<<grid, 64, 0, stream>>>(m);
    else merge_kernel<BFloat, false><<<grid, 64, 0, stream>>>(m);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PKV_ERR_LAUNCH, "merge launch failed: %s", hipGetErrorString(e));
  return PKV_OK;
}

// Internal split count wanted by a direct (num_splits == 1) launch.  One decode workgroup
// per (row, kv head) streams at most ~37 GB/s (one MI355X CU with 8 waves of one tile
// each), so with few rows the op is split into about 256 units of at least 2 tiles, merged
// by the merge kernel from partial states kept in the caller's workspace.  (2-tile units
// are streamed by one wave each; measured on C1: 10.0 us against 10.5 us for 4-tile units
// and 11.5 us for 8-tile ones.)  PKV_DIRECT_SPLIT=0 keeps the single launch.
int direct_splits_wanted(int batch, int hkv, int context) {
  static const bool on = [] {
    const char* e = getenv("PKV_DIRECT_SPLIT");
    return !(e && e[0] == '0');
  }();
  const long units = (long)batch * hkv;
  if (!on || units <= 0 || units >= 128) return 1;
  const int tiles = (context + kTile - 1) / kTile;
  long s = (256 + units - 1) / units;
  if (s > tiles / 2) s = tiles / 2;
  return s >= 2 ? (int)s : 1;
}

// The internal split a direct launch runs with: the wanted one, reduced to what the
// caller's workspace holds (no split when it holds fewer than two partial states per
// head).  The library allocates nothing for it.
int direct_splits(const Geometry& g, int context, size_t ws_bytes) {
  long s = direct_splits_wanted(g.batch, g.hkv, context);
  const size_t per_split = (size_t)g.batch * g.hq * (kD + 2) * sizeof(float);
  if (per_split == 0) return 1;
  if ((size_t)s * per_split > ws_bytes) s = (long)(ws_bytes / per_split);
  return s >= 2 ? (int)s : 1;
}

// Internal sub-splits per caller split wanted by a split launch of few units.  A launch of
// B * Hkv * S units fewer than the CUs leaves CUs idle (B = 1, Hkv = 8, S = 16: 128 of 256
// CUs), so each caller split is cut into k sub-splits, to about one unit per CU with at
// least 2 tiles each; the merge folds all S * k partial states of a head.  More than one
// unit per CU is slower (measured on C3 at 32k: 27.8 us with 256 units, 32.2 us with 512;
// B1 G4 32k with S = 16: 38.4 us with 128 units, 28.3 us with 256, 29.4 us with 512).
int split_factor_wanted(int batch, int hkv, int context, int num_splits) {
  static const bool on = [] {
    const char* e = getenv("PKV_SPLIT_SUBDIVIDE");
    return !(e && e[0] == '0');
  }();
  const long units = (long)batch * hkv * num_splits;
  const long cus = cu_count();
  if (!on || units <= 0 || num_splits <= 1 || 4 * units >= 3 * cus) return 1;
  const long tiles = (context + kTile - 1) / kTile;
  long k = (cus + units - 1) / units;
  while (k > 1 && num_splits * k * 2 > tiles) --k;
  return (int)k;
}

DecodeArgs base_args(const Geometry& g, const void* q, int q_rows, const void* k, const void* v,
                     const int32_t* table, void* out, int out_rows) {
  DecodeArgs a = {};
  a.q = (const uint8_t*)q;
  a.k_pages = (const uint8_t*)k;
  a.v_pages = (const uint8_t*)v;
  a.block_table = table;
  a.out = (uint8_t*)out;
  a.batch = g.batch;
  a.hq = g.hq;
  a.hkv = g.hkv;
  a.group = g.hq / g.hkv;
  a.q_rows = q_rows;
  a.out_rows = out_rows;
  a.page_size = g.page_size;
  a.page_shift = log2_exact(g.page_size);
  a.max_pages = g.max_pages;
  a.num_pages = g.num_pages;
  a.kv_div = 1;
  a.score_scale = kScaleLog2;
  a.v_scale = 1.0f;
  return a;
}

// How a grid op runs: one direct launch (splits == 1) or a split decode over `splits`
// sequence splits plus the merge, with partial states in `ws`.
struct GridPlan {
  int splits;
  void* ws;
};

// The partial states are written and read with 8- and 16-byte vector accesses (and the
// balanced schedule's plan entries with 16-byte ones at 16-byte offsets), so a workspace
// must be 16-byte aligned, as every torch allocation is.
int check_workspace_alignment(const void* ws) {
  if (ws && ((uintptr_t)ws & 15))
    return fail(PKV_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  return PKV_OK;
}

// Chooses the launches of a grid op and checks the workspace, before anything is launched
// (cuh:929-974 persistentkv_launch).  `internal_split` lets a launch of few units split
// itself further into the caller's workspace when it is large enough: a direct launch
// into about 256 units, a split launch into sub-splits of the caller's.
int plan_grid(const Geometry& g, const DecodeArgs& a, void* ws, size_t ws_bytes, int num_splits,
              bool internal_split, GridPlan& plan) {
  plan.splits = num_splits;
  plan.ws = ws;
  const int st = check_workspace_alignment(ws);
  if (st != PKV_OK) return st;
  if (num_splits == 1) {
    plan.splits = internal_split && ws ? direct_splits(g, a.context, ws_bytes) : 1;
    return PKV_OK;
  }
  const size_t need = pkv_workspace_bytes(g.batch, g.hq, num_splits);
  if (!ws || ws_bytes < need)
    return fail(PKV_ERR_WORKSPACE_TOO_SMALL, "split dispatch requires a workspace of %zu bytes (got %zu)",
                need, ws ? ws_bytes : (size_t)0);
  // Sub-splits of a few-unit launch, as many as the workspace holds (the caller's S alone
  // with the reference's workspace size, whose partial states then keep its layout).
  int k = internal_split ? split_factor_wanted(g.batch, g.hkv, a.context, num_splits) : 1;
  while (k > 1 && pkv_workspace_bytes(g.batch, g.hq, num_splits * k) > ws_bytes) --k;
  plan.splits = num_splits * k;
  return PKV_OK;
}

// Launches a planned grid op.
int launch_grid(const Geometry& g, DecodeArgs a, const GridPlan& plan, hipStream_t stream) {
  int st;
  const int units = (int)((long)a.batch * a.hkv);
  const int num_splits = plan.splits;
  a.num_splits = num_splits;
  if (num_splits == 1) {
    st = dispatch_decode<kDirect>(a, g.dtype, units, stream);
    return st == PKV_OK ? ok() : st;
  }
  const long states = (long)g.batch * g.hq * num_splits;
  a.part_m = (float*)plan.ws;
  a.part_l = a.part_m + states;
  a.part_acc = a.part_l + states;
  st = dispatch_decode<kSplit>(a, g.dtype, units * num_splits, stream);
  if (st != PKV_OK) return st;
  MergeArgs m = {};
  m.part_m = a.part_m;
  m.part_l = a.part_l;
  m.part_acc = a.part_acc;
  m.out_indices = a.out_indices;
  m.out = a.out;
  m.batch = g.batch;
  m.hq = g.hq;
  m.out_rows = a.out_rows;
  m.num_splits = num_splits;
  st = dispatch_merge(m, false, g.dtype, stream);
  return st == PKV_OK ? ok() : st;
}

// K/V storage of a launch: 2-byte (the activation dtype) or fp8 (OCP e4m3) with per-tensor
// dequantisation scales, K = k_scale * k8 and V = v_scale * v8.
struct KvQuant {
  bool fp8 = false;
  float k_scale = 1.0f, v_scale = 1.0f;
};

int check_quant(const Geometry& g, const KvQuant& kq) {
  if (!kq.fp8) return PKV_OK;
  if (g.page_size % 16 != 0)
    return fail(PKV_ERR_UNSUPPORTED, "fp8 K/V requires page_size to be a multiple of 16 (got %d)",
                g.page_size);
  if (!(kq.k_scale > 0.f) || !std::isfinite(kq.k_scale) || !std::isfinite(kq.v_scale))
    return fail(PKV_ERR_INVALID_ARGUMENT, "k_scale must be positive and finite and v_scale finite");
  return PKV_OK;
}

void apply_quant(DecodeArgs& a, const KvQuant& kq) {
  a.kv_fp8 = kq.fp8 ? 1 : 0;
  a.score_scale = kScaleLog2 * kq.k_scale;
  a.v_scale = kq.v_scale;
}

// Each row's newest token for the *_append ops ([B, Hkv, 128] in the KV dtype), or null.
struct NewToken {
  const void* k = nullptr;
  const void* v = nullptr;
};

// The fused append of the *_append ops.  2-byte pools with pages that are multiples of
// 16 take the new token inside the decode (AppendPager).  Other page sizes, and fp8
// pools, run the append kernel first on the same stream: an in-decode fp8 variant (the
// e4m3 encode on the reloaded lanes) measured slower than the two launches.
// check_new_token validates the arguments without launching anything; apply_new_token
// (after apply_quant and after every other check of the op) launches or wires the append.
int check_new_token(const DecodeArgs& a, const NewToken& nt) {
  if (!nt.k && !nt.v) return PKV_OK;
  if (!nt.k || !nt.v) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new and v_new must both be set");
  if (!a.seq_lens) return fail(PKV_ERR_INVALID_ARGUMENT, "the fused append needs seq_lens");
  return PKV_OK;
}

int apply_new_token(const Geometry& g, DecodeArgs& a, const NewToken& nt, const KvQuant& kq,
                    hipStream_t stream) {
  if (!nt.k && !nt.v) return PKV_OK;
  if (a.kv_fp8)
    return pkv_append_kv_fp8(nt.k, nt.v, const_cast<uint8_t*>(a.k_pages),
                             const_cast<uint8_t*>(a.v_pages), a.block_table, a.seq_lens, g.batch,
                             g.hkv, kD, g.num_pages, g.page_size, g.max_pages, kq.k_scale,
                             kq.v_scale, g.dtype, stream);
  if (g.page_size % 16 == 0) {
    a.k_new = (const uint8_t*)nt.k;
    a.v_new = (const uint8_t*)nt.v;
    return PKV_OK;
  }
  return pkv_append_kv(nt.k, nt.v, const_cast<uint8_t*>(a.k_pages), const_cast<uint8_t*>(a.v_pages),
                       a.block_table, a.seq_lens, g.batch, g.hkv, kD, g.num_pages, g.page_size,
                       g.max_pages, g.dtype, stream);
}

// Shared body of the three paged grid ops.
int run_grid(const Geometry& g, const void* q, int q_rows, const void* k, const void* v,
             const int32_t* table, const int32_t* seq_lens, const int32_t* q_idx,
             const int32_t* out_idx, void* out, int out_rows, void* ws, size_t ws_bytes,
             int context, int num_splits, void* stream_ptr, const KvQuant& kq = KvQuant{},
             const NewToken& nt = NewToken{}) {
  int st = check_geometry(g, q, k, v, table, out);
  if (st != PKV_OK) return st;
  st = check_quant(g, kq);
  if (st != PKV_OK) return st;
  if (context <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "context must be positive");
  if (num_splits <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "num_splits must be positive");
  const int total_tiles = (context + kTile - 1) / kTile;
  if (num_splits > total_tiles)  // cuh:1042-1043
    return fail(PKV_ERR_INVALID_ARGUMENT, "num_splits=%d exceeds ceil(context/32)=%d", num_splits,
                total_tiles);
  if ((long)g.max_pages * g.page_size < context)  // cuh:1131
    return fail(PKV_ERR_INVALID_ARGUMENT, "block_table has %d pages of %d tokens, fewer than context=%d",
                g.max_pages, g.page_size, context);
  if (q_rows <= 0 && g.batch > 0) return fail(PKV_ERR_INVALID_ARGUMENT, "q has no rows");
  if (g.batch == 0) return ok();
  DecodeArgs a = base_args(g, q, q_rows, k, v, table, out, out_rows);
  a.seq_lens = seq_lens;
  a.q_indices = q_idx;
  a.out_indices = out_idx;
  a.context = context;
  apply_quant(a, kq);
  st = check_new_token(a, nt);
  if (st != PKV_OK) return st;
  GridPlan plan;
  st = plan_grid(g, a, ws, ws_bytes, num_splits, true, plan);
  if (st != PKV_OK) return st;
  // Every argument is checked: only now may the append write the pools.
  st = apply_new_token(g, a, nt, kq, (hipStream_t)stream_ptr);
  if (st != PKV_OK) return st;
  return launch_grid(g, a, plan, (hipStream_t)stream_ptr);
}

// Contiguous K/V [B, Hkv, N, 128] (cuh:128-178).  `baseline` runs one unit per query
// head that streams its own KV head, as the reference's query-head baseline does
// (cuh:786-889): virtual Hkv = Hq with kv_div = G, one launch, no split.
int run_contiguous(const Geometry& g, const void* q, const void* k, const void* v, void* out,
                   void* ws, size_t ws_bytes, int context, int num_splits, bool baseline,
                   void* stream_ptr) {
  if (context <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "N must be positive");
  Geometry checked = g;  // no pages: only the head and pointer checks apply
  checked.page_size = 16;
  checked.num_pages = 1;
  checked.max_pages = 1;
  int st = check_geometry(checked, q, k, v, (const void*)1, out);
  if (st != PKV_OK) return st;
  if (num_splits <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "num_splits must be positive");
  const int total_tiles = (context + kTile - 1) / kTile;
  if (num_splits > total_tiles)  // cuh:1042-1043
    return fail(PKV_ERR_INVALID_ARGUMENT, "num_splits=%d exceeds ceil(context/32)=%d", num_splits,
                total_tiles);
  if (g.batch == 0) return ok();
  DecodeArgs a = base_args(g, q, g.batch, k, v, nullptr, out, g.batch);
  a.context = context;
  a.page_size = context;
  if (baseline) {
    a.kv_div = a.group;
    a.hkv = g.hq;
    a.group = 1;
  }
  GridPlan plan;
  st = plan_grid(g, a, ws, ws_bytes, num_splits, !baseline, plan);
  if (st != PKV_OK) return st;
  return launch_grid(g, a, plan, (hipStream_t)stream_ptr);
}

struct QueueCall {
  Geometry g;
  const void *q, *k, *v;
  int q_rows;
  const int32_t *table, *seq_lens, *items, *offsets, *q_idx, *out_idx;
  int32_t* counters;
  void* out;
  int out_rows;
  void* ws;
  size_t ws_bytes;
  int bucket_context, num_tasks, total_slots;
};

int check_queue(const QueueCall& c, bool need_out) {
  int st = check_geometry(c.g, c.q, c.k, c.v, c.table, need_out ? c.out : (const void*)1);
  if (st != PKV_OK) return st;
  if (c.bucket_context <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "bucket_context must be positive");
  if (c.num_tasks <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "work_items must not be empty");
  if (c.total_slots <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "total_partial_slots must be positive");
  if (!c.items || !c.offsets || !c.seq_lens)
    return fail(PKV_ERR_INVALID_ARGUMENT, "work-queue metadata pointer is null");
  if (c.q_rows <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "q_source has no rows");
  const size_t need = pkv_workqueue_workspace_bytes(c.total_slots, c.g.hq);
  if (!c.ws || c.ws_bytes < need)
    return fail(PKV_ERR_WORKSPACE_TOO_SMALL, "work-queue dispatch requires a workspace of %zu bytes (got %zu)",
                need, c.ws ? c.ws_bytes : (size_t)0);
  return check_workspace_alignment(c.ws);
}

DecodeArgs queue_args(const QueueCall& c) {
  DecodeArgs a = base_args(c.g, c.q, c.q_rows, c.k, c.v, c.table, c.out, c.out_rows);
  a.seq_lens = c.seq_lens;
  a.q_indices = c.q_idx;
  a.out_indices = c.out_idx;
  a.work_items = c.items;
  a.split_offsets = c.offsets;
  a.context = c.bucket_context;
  a.num_tasks = c.num_tasks;
  a.total_slots = c.total_slots;
  const long states = (long)c.total_slots * c.g.hq;
  a.part_m = (float*)c.ws;
  a.part_l = a.part_m + states;
  a.part_acc = a.part_l + states;
  return a;
}

MergeArgs queue_merge_args(const DecodeArgs& a) {
  MergeArgs m = {};
  m.part_m = a.part_m;
  m.part_l = a.part_l;
  m.part_acc = a.part_acc;
  m.seq_lens = a.seq_lens;
  m.split_offsets = a.split_offsets;
  m.out_indices = a.out_indices;
  m.out = a.out;
  m.batch = a.batch;
  m.hq = a.hq;
  m.out_rows = a.out_rows;
  m.total_slots = a.total_slots;
  m.num_tasks = a.num_tasks;
  m.hkv = a.hkv;
  m.max_tokens = (int)((long)a.max_pages * a.page_size > 0x7fffffffL ? 0x7fffffff
                                                                     : (long)a.max_pages * a.page_size);
  return m;
}

int run_indexed(const Geometry& g, const void* q_source, int32_t q_rows, const void* k_pages,
                const void* v_pages, const int32_t* block_table, const int32_t* seq_lens,
                const int32_t* q_indices, const int32_t* out_indices, void* output,
                int32_t out_rows, void* workspace, size_t workspace_bytes, int32_t bucket_context,
                int32_t num_splits, void* stream, const KvQuant& kq,
                const NewToken& nt = NewToken{}) {
  if (g.batch > 0 && (!seq_lens || !q_indices || !out_indices))
    return fail(PKV_ERR_INVALID_ARGUMENT, "seq_lens, q_indices and out_indices must be non-null");
  if (g.batch > 0 && out_rows <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "output has no rows");
  return run_grid(g, q_source, q_rows, k_pages, v_pages, block_table, seq_lens, q_indices,
                  out_indices, output, out_rows, workspace, workspace_bytes, bucket_context,
                  num_splits, stream, kq, nt);
}

// Waves of the balanced schedule for a work-queue call (bal_waves_per_cu per CU), or 0
// when the call takes the per-item schedule: with the fused merge, with G > 16 (the
// two-head-block kernel), with page sizes that are not multiples of 16, with more than 256
// rows, or when the workspace cannot hold the layout at kBalWavesMax waves per CU (one
// threshold, pkv_workqueue_balanced_workspace_bytes, for every K/V dtype).  PKV_BALANCED=0
// keeps every call on the per-item schedule (tuning).
// Layout of the balanced schedule's workspace: (pairs + waves) * G partial states (m, l,
// acc), rounded up to an even count so that acc, at 8 bytes per state, starts on a 16-byte
// boundary (the merge reads it with 16-byte loads); then one 16-byte plan entry per
// (row, kv head) pair; then one int per decode workgroup (one per CU), its part of the
// queue check.
long balanced_states(long pairs, long waves, int G) { return ((pairs + waves) * G + 1) & ~1L; }
size_t balanced_plan_offset(long pairs, long waves, int G) {
  return (size_t)balanced_states(pairs, waves, G) * (kD + 2) * sizeof(float);
}
size_t balanced_flags_offset(long pairs, long waves, int G) {
  return balanced_plan_offset(pairs, waves, G) + (size_t)pairs * 16;
}
size_t balanced_bytes(long pairs, long waves, int G) {
  return balanced_flags_offset(pairs, waves, G) + (size_t)cu_count() * sizeof(int32_t);
}

int balanced_waves(const Geometry& g, size_t ws_bytes, int fused_merge, bool fp8) {
  static const bool on = [] {
    const char* e = getenv("PKV_BALANCED");
    return !(e && e[0] == '0');
  }();
  if (!on || fused_merge || g.hkv <= 0 || g.batch <= 0) return 0;
  const int G = g.hq / g.hkv;
  if (G > 16 || g.page_size % 16 != 0 || g.batch > 64 * kBalRowChunks) return 0;
  if (balanced_bytes((long)g.batch * g.hkv, (long)kBalWavesMax * cu_count(), G) > ws_bytes) return 0;
  return bal_waves_per_cu(fp8) * cu_count();
}

// Stages of the work-queue op: 1 = decode, 2 = merge, 3 = both (the combined op).
int run_workqueue(const QueueCall& c, int32_t fused_merge, hipStream_t stream, const KvQuant& kq,
                  const NewToken& nt = NewToken{}, int stages = 3) {
  int st = check_queue(c, true);
  if (st != PKV_OK) return st;
  st = check_quant(c.g, kq);
  if (st != PKV_OK) return st;
  if (c.out_rows <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "output has no rows");
  if (fused_merge && !c.counters) return fail(PKV_ERR_INVALID_ARGUMENT, "merge_counters is null");
  if (c.g.batch == 0) return ok();
  DecodeArgs a = queue_args(c);
  apply_quant(a, kq);
  st = check_new_token(a, nt);
  if (st != PKV_OK) return st;
  const int waves = balanced_waves(c.g, c.ws_bytes, fused_merge, kq.fp8);
  // Every argument is checked (the workspace by check_queue): the append may now run.
  if (stages & 1) {
    st = apply_new_token(c.g, a, nt, kq, stream);
    if (st != PKV_OK) return st;
  }
  if (waves > 0) {
    const long pairs = (long)c.g.batch * c.g.hkv;
    const long states = balanced_states(pairs, waves, a.group);
    a.part_m = (float*)c.ws;
    a.part_l = a.part_m + states;
    a.part_acc = a.part_l + states;
    a.bal_plan = (int32_t*)((uint8_t*)c.ws + balanced_plan_offset(pairs, waves, a.group));
    a.bal_flags = (int32_t*)((uint8_t*)c.ws + balanced_flags_offset(pairs, waves, a.group));
    const int wg_waves = bal_waves_per_cu(kq.fp8);
    const int check_wgs = waves / wg_waves;
    hipError_t e = hipSuccess;
    if (stages & 1) {
      // 96 KB of LDS per workgroup keeps one workgroup on each CU.
      const size_t lds = 96 * 1024;
      const int grid = check_wgs;
      const bool bf = c.g.dtype == PKV_DTYPE_BF16;
      if (a.kv_fp8) {
        if (bf) balanced_decode_kernel<BFloat, kPgFp8><<<grid, wg_waves * 64, lds, stream>>>(a);
        else balanced_decode_kernel<Half, kPgFp8><<<grid, wg_waves * 64, lds, stream>>>(a);
      } else if (a.k_new) {
        if (bf) balanced_decode_kernel<BFloat, kPgAppend><<<grid, wg_waves * 64, lds, stream>>>(a);
        else balanced_decode_kernel<Half, kPgAppend><<<grid, wg_waves * 64, lds, stream>>>(a);
      } else {
        if (bf) balanced_decode_kernel<BFloat, kPgFast><<<grid, wg_waves * 64, lds, stream>>>(a);
        else balanced_decode_kernel<Half, kPgFast><<<grid, wg_waves * 64, lds, stream>>>(a);
      }
      e = hipGetLastError();
      if (e != hipSuccess) return fail(PKV_ERR_LAUNCH, "decode launch failed: %s", hipGetErrorString(e));
    }
    if (stages & 2) {
      const int grid = c.g.batch * c.g.hq;
      // Waves per (row, query head): as many as the decode ran per CU (a pair's pieces
      // scale with them; C4 step 43.0 against 43.4 us with 4 after two decode waves, fp8
      // merge stage 5.9-6.2 against 6.9-7.0 us with 2 after four), at most the number that
      // keeps the grid within ~8 waves per CU.
      int merge_waves = wg_waves;
      while (merge_waves > 1 && (long)grid * merge_waves > 8L * cu_count()) merge_waves >>= 1;
      const int block = merge_waves * 64;
      // The wide fold (one round trip for up to kWideStates groups, ~250 VGPRs) where a
      // merge wave's share can exceed one chunk: few pairs per merge wave.
      const bool wide = (long)c.g.batch * c.g.hkv * merge_waves * kMergeChunk < waves;
      const bool bf = c.g.dtype == PKV_DTYPE_BF16;
      // The pager of the merge's fallback: fp8 pages, else 2-byte pages (with the fused
      // append the decode has already written the new token).
      if (a.kv_fp8) {
        if (wide) {
          if (bf) balanced_merge_kernel<BFloat, true, kPgFp8><<<grid, block, 0, stream>>>(a, waves, check_wgs);
          else balanced_merge_kernel<Half, true, kPgFp8><<<grid, block, 0, stream>>>(a, waves, check_wgs);
        } else {
          if (bf) balanced_merge_kernel<BFloat, false, kPgFp8><<<grid, block, 0, stream>>>(a, waves, check_wgs);
          else balanced_merge_kernel<Half, false, kPgFp8><<<grid, block, 0, stream>>>(a, waves, check_wgs);
        }
      } else if (wide) {
        if (bf) balanced_merge_kernel<BFloat, true, kPgFast><<<grid, block, 0, stream>>>(a, waves, check_wgs);
        else balanced_merge_kernel<Half, true, kPgFast><<<grid, block, 0, stream>>>(a, waves, check_wgs);
      } else {
        if (bf) balanced_merge_kernel<BFloat, false, kPgFast><<<grid, block, 0, stream>>>(a, waves, check_wgs);
        else balanced_merge_kernel<Half, false, kPgFast><<<grid, block, 0, stream>>>(a, waves, check_wgs);
      }
      e = hipGetLastError();
      if (e != hipSuccess) return fail(PKV_ERR_LAUNCH, "merge launch failed: %s", hipGetErrorString(e));
    }
    return ok();
  }
  a.merge_counters = fused_merge ? c.counters : nullptr;
  if (stages & 1) {
    st = dispatch_decode<kQueue>(a, c.g.dtype, c.num_tasks, stream);
    if (st != PKV_OK) return st;
  }
  if (!fused_merge && (stages & 2)) {
    st = dispatch_merge(queue_merge_args(a), true, c.g.dtype, stream);
    if (st != PKV_OK) return st;
  }
  return ok();
}

// Stage 1 of the work-queue op: the decode kernel alone.
int run_queue_decode(const QueueCall& c, hipStream_t stream, const KvQuant& kq) {
  int st = check_queue(c, false);
  if (st != PKV_OK) return st;
  st = check_quant(c.g, kq);
  if (st != PKV_OK) return st;
  if (c.g.batch == 0) return ok();
  DecodeArgs a = queue_args(c);
  apply_quant(a, kq);
  st = dispatch_decode<kQueue>(a, c.g.dtype, c.num_tasks, stream);
  return st == PKV_OK ? ok() : st;
}

// ---------------------------------------------------------------------------------
// Static scratch of the allocation-free work-queue entry point: the partial states of
// one call, in device memory that the code object brings with it (each GPU the library
// runs on holds its own copy until the process ends).  On the host, `scratch` names a
// host-side stand-in, never the device array: its device address comes from
// hipGetSymbolAddress, taken once per device on that device's first call, and only that
// address is passed to kernels.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU (other streams, concurrent graph replays) race.  The work-queue
// op needs no part of it cleared: every partial state it merges is written by the same
// call first, and the slots of empty splits are skipped, not read.
// ---------------------------------------------------------------------------------
constexpr size_t kScratchBytes = 16u << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` on the current device, or null (with the error set).
void* scratch_address() {
  static std::mutex mu;
  static void* address[64] = {};
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
    (void)hipGetLastError();
    fail(PKV_ERR_LAUNCH, "no current HIP device for the static scratch");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!address[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      fail(PKV_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
           hipGetErrorString(e));
      return nullptr;
    }
    address[device] = p;
  }
  return address[device];
}

}  // namespace pkv

using namespace pkv;

extern "C" {

const char* pkv_last_error(void) { return g_error; }

const char* pkv_status_string(int status) {
  switch (status) {
    case PKV_OK: return "PKV_OK";
    case PKV_ERR_INVALID_ARGUMENT: return "PKV_ERR_INVALID_ARGUMENT";
    case PKV_ERR_UNSUPPORTED: return "PKV_ERR_UNSUPPORTED";
    case PKV_ERR_WORKSPACE_TOO_SMALL: return "PKV_ERR_WORKSPACE_TOO_SMALL";
    case PKV_ERR_LAUNCH: return "PKV_ERR_LAUNCH";
    case PKV_ERR_CAPACITY: return "PKV_ERR_CAPACITY";
    default: return "PKV_ERR_UNKNOWN";
  }
}

int pkv_version(void) { return 100; }

size_t pkv_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_splits) {
  if (num_splits <= 1 || batch <= 0 || num_q_heads <= 0) return 0;
  return (size_t)batch * num_q_heads * num_splits * (kD + 2) * sizeof(float);
}

size_t pkv_workqueue_workspace_bytes(int32_t total_partial_slots, int32_t num_q_heads) {
  if (total_partial_slots <= 0 || num_q_heads <= 0) return 0;
  return (size_t)total_partial_slots * num_q_heads * (kD + 2) * sizeof(float);
}

size_t pkv_direct_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t context) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || context <= 0) return 0;
  const int s = direct_splits_wanted(batch, num_kv_heads, context);
  return s > 1 ? pkv_workspace_bytes(batch, num_q_heads, s) : 0;
}

size_t pkv_split_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                 int32_t context, int32_t num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || context <= 0 || num_splits <= 1)
    return 0;
  const int k = split_factor_wanted(batch, num_kv_heads, context, num_splits);
  return pkv_workspace_bytes(batch, num_q_heads, num_splits * k);
}

int pkv_paged_attention(const void* q, const void* k_pages, const void* v_pages,
                        const int32_t* block_table, void* output, void* workspace,
                        size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t num_pages,
                        int32_t page_size, int32_t max_pages, int32_t context,
                        int32_t num_splits, int32_t dtype, void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  return run_grid(g, q, batch, k_pages, v_pages, block_table, nullptr, nullptr, nullptr, output,
                  batch, workspace, workspace_bytes, context, num_splits, stream);
}

int pkv_paged_attention_masked(const void* q, const void* k_pages, const void* v_pages,
                               const int32_t* block_table, const int32_t* seq_lens, void* output,
                               void* workspace, size_t workspace_bytes, int32_t batch,
                               int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t num_pages, int32_t page_size, int32_t max_pages,
                               int32_t bucket_context, int32_t num_splits, int32_t dtype,
                               void* stream) {
  if (batch > 0 && !seq_lens) return fail(PKV_ERR_INVALID_ARGUMENT, "seq_lens is null");
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  return run_grid(g, q, batch, k_pages, v_pages, block_table, seq_lens, nullptr, nullptr, output,
                  batch, workspace, workspace_bytes, bucket_context, num_splits, stream);
}

int pkv_paged_attention_indexed(const void* q_source, int32_t q_rows, const void* k_pages,
                                const void* v_pages, const int32_t* block_table,
                                const int32_t* seq_lens, const int32_t* q_indices,
                                const int32_t* out_indices, void* output, int32_t out_rows,
                                void* workspace, size_t workspace_bytes, int32_t batch,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t num_pages, int32_t page_size, int32_t max_pages,
                                int32_t bucket_context, int32_t num_splits, int32_t dtype,
                                void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  return run_indexed(g, q_source, q_rows, k_pages, v_pages, block_table, seq_lens, q_indices,
                     out_indices, output, out_rows, workspace, workspace_bytes, bucket_context,
                     num_splits, stream, KvQuant{});
}

int pkv_paged_attention_indexed_fp8(const void* q_source, int32_t q_rows, const void* k_pages,
                                    const void* v_pages, const int32_t* block_table,
                                    const int32_t* seq_lens, const int32_t* q_indices,
                                    const int32_t* out_indices, void* output, int32_t out_rows,
                                    void* workspace, size_t workspace_bytes, int32_t batch,
                                    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t num_pages, int32_t page_size, int32_t max_pages,
                                    int32_t bucket_context, int32_t num_splits, float k_scale,
                                    float v_scale, int32_t dtype, void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  return run_indexed(g, q_source, q_rows, k_pages, v_pages, block_table, seq_lens, q_indices,
                     out_indices, output, out_rows, workspace, workspace_bytes, bucket_context,
                     num_splits, stream, KvQuant{true, k_scale, v_scale});
}

int pkv_attention_contiguous(const void* q, const void* k, const void* v, void* output,
                             void* workspace, size_t workspace_bytes, int32_t batch,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t context,
                             int32_t head_dim, int32_t num_splits, int32_t dtype, void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, 1, 16, 1, dtype};
  return run_contiguous(g, q, k, v, output, workspace, workspace_bytes, context, num_splits, false,
                        stream);
}

int pkv_attention_query_head_baseline(const void* q, const void* k, const void* v, void* output,
                                      int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                      int32_t context, int32_t head_dim, int32_t dtype,
                                      void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, 1, 16, 1, dtype};
  return run_contiguous(g, q, k, v, output, nullptr, 0, context, 1, true, stream);
}

int pkv_paged_attention_workqueue(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices, void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
    int32_t max_pages, int32_t bucket_context, int32_t total_partial_slots,
    int32_t fused_merge, int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, merge_counters, output, out_rows,
                    workspace, workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  return run_workqueue(c, fused_merge, (hipStream_t)stream, KvQuant{});
}

int pkv_paged_attention_workqueue_stage(
    int32_t stage, const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, const int32_t* q_indices,
    const int32_t* out_indices, void* output, int32_t out_rows, void* workspace,
    size_t workspace_bytes, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t total_partial_slots, int32_t kv_fp8, float k_scale,
    float v_scale, int32_t dtype, void* stream) {
  if (stage != 1 && stage != 2) return fail(PKV_ERR_INVALID_ARGUMENT, "stage must be 1 or 2");
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, nullptr, output, out_rows,
                    workspace, workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  const KvQuant kq = kv_fp8 ? KvQuant{true, k_scale, v_scale} : KvQuant{};
  return run_workqueue(c, 0, (hipStream_t)stream, kq, NewToken{}, stage);
}

size_t pkv_workqueue_balanced_workspace_bytes(int32_t batch, int32_t num_q_heads,
                                              int32_t num_kv_heads) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      num_q_heads / num_kv_heads > 16 || batch > 64 * kBalRowChunks)
    return 0;  // sizes the balanced schedule never takes
  const long waves = (long)kBalWavesMax * cu_count();
  return balanced_bytes((long)batch * num_kv_heads, waves, num_q_heads / num_kv_heads);
}

int pkv_workqueue_schedule(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t page_size, size_t workspace_bytes, int32_t fused_merge) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      page_size <= 0)
    return 0;
  const Geometry g{batch, num_q_heads, num_kv_heads, kD, 1, page_size, 1, PKV_DTYPE_F16};
  return balanced_waves(g, workspace_bytes, fused_merge, false) > 0 ? 1 : 0;
}

int pkv_paged_attention_workqueue_noalloc(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices, void* output, int32_t out_rows,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t num_pages,
    int32_t page_size, int32_t max_pages, int32_t bucket_context, int32_t total_partial_slots,
    int32_t fused_merge, int32_t dtype, void* stream) {
  const size_t need = pkv_workqueue_workspace_bytes(total_partial_slots, num_q_heads);
  if (need > kScratchBytes)
    return fail(PKV_ERR_WORKSPACE_TOO_SMALL,
                "the partial states of %d slots x %d heads need %zu bytes, more than the %zu-byte "
                "static scratch of pkv_paged_attention_workqueue_noalloc",
                total_partial_slots, num_q_heads, need, kScratchBytes);
  void* ws = scratch_address();
  if (!ws) return PKV_ERR_LAUNCH;
  // The scratch stands in for a workspace of exactly `need` bytes, so the call takes the
  // schedule that a caller with the reference-sized workspace gets.
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, merge_counters, output, out_rows,
                    ws, need, bucket_context, num_tasks, total_partial_slots};
  return run_workqueue(c, fused_merge, (hipStream_t)stream, KvQuant{});
}

int pkv_paged_attention_masked_append(
    const void* q, const void* k_pages, const void* v_pages, const int32_t* block_table,
    const int32_t* seq_lens, void* output, void* workspace, size_t workspace_bytes,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t num_pages, int32_t page_size, int32_t max_pages, int32_t bucket_context,
    int32_t num_splits, const void* k_new, const void* v_new, int32_t dtype, void* stream) {
  if (batch > 0 && !seq_lens) return fail(PKV_ERR_INVALID_ARGUMENT, "seq_lens is null");
  if (batch > 0 && (!k_new || !v_new)) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new or v_new is null");
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  return run_grid(g, q, batch, k_pages, v_pages, block_table, seq_lens, nullptr, nullptr, output,
                  batch, workspace, workspace_bytes, bucket_context, num_splits, stream, KvQuant{},
                  NewToken{k_new, v_new});
}

int pkv_paged_attention_indexed_append(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* q_indices,
    const int32_t* out_indices, void* output, int32_t out_rows, void* workspace,
    size_t workspace_bytes, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, const void* k_new, const void* v_new,
    int32_t dtype, void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  if (batch > 0 && (!k_new || !v_new)) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new or v_new is null");
  return run_indexed(g, q_source, q_rows, k_pages, v_pages, block_table, seq_lens, q_indices,
                     out_indices, output, out_rows, workspace, workspace_bytes, bucket_context,
                     num_splits, stream, KvQuant{}, NewToken{k_new, v_new});
}

int pkv_paged_attention_workqueue_append(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices, void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
    int32_t max_pages, int32_t bucket_context, int32_t total_partial_slots,
    int32_t fused_merge, const void* k_new, const void* v_new, int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, merge_counters, output, out_rows,
                    workspace, workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  if (batch > 0 && (!k_new || !v_new)) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new or v_new is null");
  return run_workqueue(c, fused_merge, (hipStream_t)stream, KvQuant{}, NewToken{k_new, v_new});
}

int pkv_paged_attention_indexed_fp8_append(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* q_indices,
    const int32_t* out_indices, void* output, int32_t out_rows, void* workspace,
    size_t workspace_bytes, int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t num_pages, int32_t page_size, int32_t max_pages,
    int32_t bucket_context, int32_t num_splits, float k_scale, float v_scale,
    const void* k_new, const void* v_new, int32_t dtype, void* stream) {
  const Geometry g{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype};
  if (batch > 0 && (!k_new || !v_new)) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new or v_new is null");
  return run_indexed(g, q_source, q_rows, k_pages, v_pages, block_table, seq_lens, q_indices,
                     out_indices, output, out_rows, workspace, workspace_bytes, bucket_context,
                     num_splits, stream, KvQuant{true, k_scale, v_scale}, NewToken{k_new, v_new});
}

int pkv_paged_attention_workqueue_fp8_append(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices, void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
    int32_t max_pages, int32_t bucket_context, int32_t total_partial_slots,
    int32_t fused_merge, float k_scale, float v_scale, const void* k_new, const void* v_new,
    int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, merge_counters, output, out_rows,
                    workspace, workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  if (batch > 0 && (!k_new || !v_new)) return fail(PKV_ERR_INVALID_ARGUMENT, "k_new or v_new is null");
  return run_workqueue(c, fused_merge, (hipStream_t)stream, KvQuant{true, k_scale, v_scale},
                       NewToken{k_new, v_new});
}

int pkv_paged_attention_workqueue_fp8(
    const void* q_source, int32_t q_rows, const void* k_pages, const void* v_pages,
    const int32_t* block_table, const int32_t* seq_lens, const int32_t* work_items,
    int32_t num_tasks, const int32_t* split_offsets, int32_t* merge_counters,
    const int32_t* q_indices, const int32_t* out_indices, void* output, int32_t out_rows,
    void* workspace, size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t num_pages, int32_t page_size,
    int32_t max_pages, int32_t bucket_context, int32_t total_partial_slots,
    int32_t fused_merge, float k_scale, float v_scale, int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, out_indices, merge_counters, output, out_rows,
                    workspace, workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  return run_workqueue(c, fused_merge, (hipStream_t)stream, KvQuant{true, k_scale, v_scale});
}

int pkv_workqueue_decode(const void* q_source, int32_t q_rows, const void* k_pages,
                         const void* v_pages, const int32_t* block_table, const int32_t* seq_lens,
                         const int32_t* work_items, int32_t num_tasks,
                         const int32_t* split_offsets, const int32_t* q_indices, void* workspace,
                         size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t num_pages,
                         int32_t page_size, int32_t max_pages, int32_t bucket_context,
                         int32_t total_partial_slots, int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, nullptr, nullptr, nullptr, 0, workspace,
                    workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  return run_queue_decode(c, (hipStream_t)stream, KvQuant{});
}

int pkv_workqueue_decode_fp8(const void* q_source, int32_t q_rows, const void* k_pages,
                             const void* v_pages, const int32_t* block_table,
                             const int32_t* seq_lens, const int32_t* work_items, int32_t num_tasks,
                             const int32_t* split_offsets, const int32_t* q_indices,
                             void* workspace, size_t workspace_bytes, int32_t batch,
                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t num_pages, int32_t page_size, int32_t max_pages,
                             int32_t bucket_context, int32_t total_partial_slots, float k_scale,
                             float v_scale, int32_t dtype, void* stream) {
  const QueueCall c{{batch, num_q_heads, num_kv_heads, head_dim, num_pages, page_size, max_pages, dtype},
                    q_source, k_pages, v_pages, q_rows, block_table, seq_lens, work_items,
                    split_offsets, q_indices, nullptr, nullptr, nullptr, 0, workspace,
                    workspace_bytes, bucket_context, num_tasks, total_partial_slots};
  return run_queue_decode(c, (hipStream_t)stream, KvQuant{true, k_scale, v_scale});
}

int pkv_workqueue_merge(const int32_t* seq_lens, const int32_t* split_offsets,
                        const int32_t* out_indices, void* output, int32_t out_rows,
                        const void* workspace, size_t workspace_bytes, int32_t batch,
                        int32_t num_q_heads, int32_t total_partial_slots, int32_t num_tasks,
                        int32_t num_kv_heads, int32_t dtype, void* stream) {
  if (dtype != PKV_DTYPE_F16 && dtype != PKV_DTYPE_BF16)
    return fail(PKV_ERR_UNSUPPORTED, "dtype must be fp16 or bf16");
  if (batch < 0 || num_q_heads <= 0) return fail(PKV_ERR_INVALID_ARGUMENT, "bad batch or head count");
  if (num_tasks >= 0 && num_kv_heads <= 0)
    return fail(PKV_ERR_INVALID_ARGUMENT, "num_kv_heads must be positive when num_tasks is given");
  if (total_partial_slots <= 0)
    return fail(PKV_ERR_INVALID_ARGUMENT, "total_partial_slots must be positive");
  if (batch > 0 && (!seq_lens || !split_offsets || !output || out_rows <= 0))
    return fail(PKV_ERR_INVALID_ARGUMENT, "merge metadata or output is missing");
  const size_t need = pkv_workqueue_workspace_bytes(total_partial_slots, num_q_heads);
  if (!workspace || workspace_bytes < need)
    return fail(PKV_ERR_WORKSPACE_TOO_SMALL, "merge requires a workspace of %zu bytes", need);
  if (check_workspace_alignment(workspace) != PKV_OK) return PKV_ERR_INVALID_ARGUMENT;
  if (batch == 0) return ok();
  const long states = (long)total_partial_slots * num_q_heads;
  MergeArgs m = {};
  m.part_m = (const float*)workspace;
  m.part_l = m.part_m + states;
  m.part_acc = m.part_l + states;
  m.seq_lens = seq_lens;
  m.split_offsets = split_offsets;
  m.out_indices = out_indices;
  m.out = (uint8_t*)output;
  m.batch = batch;
  m.hq = num_q_heads;
  m.out_rows = out_rows;
  m.total_slots = total_partial_slots;
  m.max_tokens = 0x7fffffff;
  m.num_tasks = num_tasks < 0 ? -1 : num_tasks;
  m.hkv = num_kv_heads;
  const int st = dispatch_merge(m, true, dtype, (hipStream_t)stream);
  return st == PKV_OK ? ok() : st;
}

}  // extern "C"
