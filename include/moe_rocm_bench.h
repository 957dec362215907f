/*
 * moe_rocm_bench.h -- bench and test support exported by libmoe_rocm.so.
 *
 * Not part of the drop-in ABI of include/moe_rocm.h and without a counterpart in
 * the reference: synthetic weight generation and the measurement probes that
 * bench.py and the tests use. A backend user never needs these.
 */
#ifndef MOE_ROCM_BENCH_H
#define MOE_ROCM_BENCH_H

#include "moe_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic inputs ------------------------------------------------------ */
/* Fill device bytes with the counter-based SplitMix64 generator of
 * moe_rocm/synth.py: MXFP4 blocks (e8m0 uniform in [119,127], nibbles uniform)
 * or Q4_K super-blocks (fp16 d ~|N(0,0.01)|, dmin ~|N(0,0.005)| by the
 * Irwin-Hall(12) construction, scale and quant bytes uniform). */
int mr_synth_blocks(mr_ctx* ctx, int ggml_type, void* dst, uint64_t n_blocks, uint64_t seed);

/* ---- measurement probes ---------------------------------------------------- */
/* A plain streaming read of nbytes (a multiple of 16) from src (16-byte aligned) by
 * n_workgroups workgroups of 256 threads: workgroup b reads its own contiguous range
 * (nbytes / n_workgroups, rounded up to 4 KiB), each thread 16-byte pieces 4 KiB apart with
 * `depth` (4, 8 or 16) loads in flight at every step; one word per workgroup is written to
 * sink [n_workgroups] u32. And an empty kernel of n_workgroups workgroups. The ceilings the
 * decode kernels are measured against: the bytes a plain stream moves per microsecond and
 * the cost of a kernel boundary. Profile names "probe_read" and "probe_empty". */
int mr_probe_read(mr_ctx* ctx, const void* src, uint64_t nbytes, uint32_t n_workgroups, uint32_t depth,
                  uint32_t* sink);
int mr_probe_empty(mr_ctx* ctx, uint32_t n_workgroups);
/* The fused MXFP4 decode kernel's gate/up access pattern as a plain read: src as rows of
 * row_bytes, tiles of 16 adjacent rows (n_tiles of them, all inside the buffer, which must stay
 * readable 16 bytes past the last row); each of the 4 waves of a workgroup streams whole tiles in
 * chunks of 204 bytes per row, fetched as 240-byte 16-byte-aligned row segments, with depth (2,
 * 4 or 8) chunks in flight; or, with depth 0x100 + S (S = 6, 12 or 23), in chunks of S K steps
 * (68 S bytes per row) one at a time, to see how the segment length moves the rate. One word per
 * workgroup goes to sink. Profile name "probe_tiles". */
/* One 4-byte read every `stride` bytes (a multiple of 4) of [src, src + nbytes) by 256 workgroups:
 * caches the range's address translations while reading almost none of its bytes. sink [256] u32
 * is written only in the rare case a folded word matches a fixed pattern. Profile name
 * "probe_touch". */
int mr_probe_touch(mr_ctx* ctx, const void* src, uint64_t nbytes, uint32_t stride, uint32_t* sink);
int mr_probe_tiles(mr_ctx* ctx, const void* src, uint32_t row_bytes, uint32_t n_tiles, uint32_t n_workgroups,
                   uint32_t depth, uint32_t* sink);
/* Flag round trips between workgroups wg_a and wg_b of one launch (wg_a != wg_b, both < 1024;
 * workgroup b runs on XCD b mod 8) through the device-coherent level, as the fused decode
 * kernels hand data between workgroups: a stores i, b polls for it and stores i back, a polls
 * for that, i = 1 .. n_round_trips (<= 100000). words: 64 device u32, cleared by the call;
 * result: 4 device u64 = device-clock ticks (100 MHz) of wg_a over the round trips, round trips
 * completed (a poll gives up after 100 ms), and the XCC_ID << 32 | HW_ID of wg_a and wg_b.
 * Profile name "probe_flags". */
int mr_probe_flags(mr_ctx* ctx, uint32_t* words, uint32_t wg_a, uint32_t wg_b, uint32_t n_round_trips,
                   unsigned long long* result);

#ifdef __cplusplus
}
#endif
#endif /* MOE_ROCM_BENCH_H */
