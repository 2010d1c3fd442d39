/*
 * pkv_probe.h — C ABI of the HBM measurement probes (libpkv_probe.so), kept apart from
 * the engine library libpkv.so: streaming kernels of known size that give the decode
 * kernel's roofline its achievable-bandwidth and per-CU figures and calibrate rocprofv3's
 * FETCH_SIZE / WRITE_SIZE counters.  They are measurement tools, not part of the engine.
 */
#ifndef PKV_PROBE_H_
#define PKV_PROBE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------------
 * HBM calibration probes (counterparts of the reference's
 * micro_benchmarks/01_hbm_bandwidth.cu:20-51 read/copy kernels).
 * ------------------------------------------------------------------------------- */

/* Reads `bytes` (a multiple of 4096, < 8 TiB) of `src` once, visiting its 4 KB chunks in
 * a permuted order with access pattern 0 (contiguous 1 KB per load instruction),
 * 1 (the decode kernel's K-operand loads: 16 rows x 64 B) or 2 (its V-operand loads:
 * 4 rows x 256 B).  `sink` receives at most one word per workgroup (2048 words). */
int pkv_probe_read(const void* src, size_t bytes, int32_t pattern, void* sink, void* stream);

/* Copies `bytes` (a multiple of 16) from src to dst with a plain grid-stride kernel. */
int pkv_probe_copy(const void* src, void* dst, size_t bytes, void* stream);

/* pkv_probe_read over `workgroups` workgroups of 8 waves, at most one per CU (each holds
 * 96 KB of LDS): with fewer workgroups than CUs it measures the read bandwidth of that
 * many CUs (sink holds `workgroups` words).  No counterpart in the reference. */
int pkv_probe_read_cus(const void* src, size_t bytes, int32_t pattern, int32_t workgroups,
                       void* sink, void* stream);

/* pkv_probe_read_cus with `waves` (4, 8 or 16) waves per workgroup, each keeping
 * `chunks_per_wave` (1, 2 or 4) 4 KB chunks in flight: read bandwidth and loaded latency
 * (bytes in flight / bandwidth) against how the bytes in flight are spread over waves.
 * Pattern 3 loads whole lines (as pattern 2) and moves each chunk through LDS into the
 * K-operand layout of pattern 1 (a bank-conflict-free XOR swizzle of 16-byte columns).
 * No counterpart in the reference. */
int pkv_probe_read_inflight(const void* src, size_t bytes, int32_t pattern, int32_t waves,
                            int32_t chunks_per_wave, int32_t workgroups, void* sink,
                            void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* PKV_PROBE_H_ */
