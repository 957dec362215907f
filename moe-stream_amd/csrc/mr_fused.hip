// mr_fused.hip -- single-launch MXFP4 MoE decode layer for gfx950 (CDNA4).
//
// One kernel per layer and token does the whole of gpu_routed_moe_forward_metal
// (metal/mod.rs:1512-1677): router GEMV + top-k, gate+up dequant-matvec with
// bias and SwiGLU, down dequant-matvec with bias and the weighted combine.
//
// Matvecs run on v_mfma_scale_f32_16x16x128_f8f6f4 with the weights fed
// straight from their native 17-byte GGUF blocks: the 16 code bytes of a block
// are the A operand of one lane (32 K values), its e8m0 byte is that lane's A
// scale (GGUF kvalue*2^(e-128) == OCP e2m1*2^(e-127)). The activation vector is
// the B operand, split into kTerms e4m3 terms (B columns 0..kTerms-1, each with
// its own e8m0 scale per 32-element block); the column sum of D is the matvec.
// Within a block, MFMA k=2j <-> GGUF element j and k=2j+1 <-> element j+16
// (byte j holds both), so no weight byte is moved or repacked.
//
// Operand layout of the 16x16x128 f8f6f4 MFMA on gfx950 (lane = 16*g + i):
//   A (fp4): row i, K [32g, 32g+32), nibble n (byte n/2, low nibble first) = K 32g+n;
//            scale_a = e8m0 of that 32-K block.
//   B (fp8): column i, bytes 0..15 = K [16g, 16g+16), bytes 16..31 = K [64+16g, +16);
//            scale_b of lane (i, g) applies to K block g = K [32g, 32g+32).
//   D:       D[4g + r][i] in element r.
//
// Three groups of workgroups share one grid:
//   [0, R)        router: one expert logit per wave; publishes it as a flagged
//                 64-bit word (logit bits, launch number + 1).
//   [R, R+ND)     down: 16 output rows and a group of four slots; wave w takes slot
//                 4 sg + w of slot group sg (routed slots, then the shared expert). Its
//                 down weights are loaded into registers before the gate/up results
//                 exist, so their HBM traffic overlaps the gate/up phase. With more than
//                 four slots the row group's slot groups write partial rows and the last
//                 of them to finish (a counter per row group) combines them.
//   [R+ND, grid)  gate/up: 32 rows of one slot, both projections; 4 waves =
//                 (gate, up) x 2 row tiles, each over the full K. The x split is
//                 built in LDS while the router runs. Epilogue: bias, SwiGLU (SiLU
//                 for the shared expert), x routing weight (the sigmoid gate for
//                 the shared expert, layer.rs:1935-1951), split into the down B image.
// Workgroups are dispatched in index order; fused_supported keeps R + ND below
// the CU count and the whole grid within 3 workgroups per CU (159 VGPRs, about
// 50 KB LDS each), so every workgroup is resident from the start and no wait
// can depend on a workgroup that has not been dispatched.
// Cross-workgroup values are written with agent-scope stores: the logits carry
// their launch flag in the same 64-bit store, so routing polls them directly; the
// down B image is announced by a monotonic counter (64 copies) bumped after the
// image stores have completed. Each workgroup keeps its own launch number (read at
// entry, stored +1 at exit), so nothing is reset between launches. Every wait is
// bounded in time (the context's wait limit); a wait that runs out sets an error word read
// at mr_sync and the launch still exits.
#include "mr_device.h"
#include "mr_internal.h"
#include "mr_fused_common.h"
#include "mr_mx_mfma.h"

#include <algorithm>
#include <type_traits>

namespace mr {

constexpr int kSteps = 23;              // K steps (4 blocks each) per wave: H, I <= 2944
constexpr int kRouterVec = 12;          // float4 pairs per lane of a router row: H <= 3072
constexpr int kRouterJ = kRouterVec / 4;  // float4s per lane of one wave's quarter of a router row
constexpr int kRouterRounds = 4;          // logits per router workgroup at most
constexpr int kImgVec = 12;             // 16-byte image loads per lane for one slot: I <= 3072


struct FusedArgs {
  ExpertLoc gate, up, down;
  const float* gate_b;
  const float* up_b;
  const float* down_b;
  const float* router_w;
  const float* router_b;
  const float* mask;
  const float* x;
  float* y;
  float* logits_out;  // router logits [E] of this launch (the layer's logits output) or null
  uint32_t* fs;   // this layer's sync block
  uint32_t* err;  // context error word (read and cleared by mr_sync)
  const uint8_t* sh_gate;  // shared expert matrices (one expert, MXFP4) or null
  const uint8_t* sh_up;
  const uint8_t* sh_down;
  const float* sh_gate_inp;
  uint8_t* dimg;  // [k * nbI + nbIsh][kImgBytes] down B image: routed slots, then the shared expert
  uint32_t* dsc;  // [k * nbI + nbIsh] 4 e8m0 bytes (one per term)
  float* dpart;   // [ktot][H] down rows of each slot (more than four slots: combined by the last slot group)
  int H, I, E, k, ktot, has_sh;
  int Ish;  // shared expert width (a multiple of 32, at most 32 * 4 * kSteps; 0 without one)
  uint32_t flags;
  int act;
  float alpha, limit;
  int R, NG, ND;
  int rr;  // logits per router workgroup (1, 2 or 4; router_rounds)
  int NS;        // down row groups split into two 8-row workgroups (CU balance; at most four slots)
  int NDR, nsl;  // row groups and slot groups of the down role (ND = NDR * nsl)
  WaitBound wb;  // time limit of the cross-workgroup waits
  int dn_delay;  // s_sleep(8) rounds before the down role's weight prefetch (dn_delay_rounds)
  int perm_nc;  // CU count of the role permutation (role_index), 0: identity
  uint32_t lds_img_bytes;     // dynamic LDS: image bytes, then 4-byte scales
  PrefetchRows pf;            // the next layer's router rows (router workgroups read them)
  const float* pf_nw;         // the next layer's norm weights (mr_layer_set_norm) or null
  NormResid nr;               // fused RMSNorm of x and residual added to y (off: nr.w == nullptr)
  unsigned long long* trace;  // MR_FUSED_TRACE builds only: [grid][16] timestamps
};

// In place, raw windows -> MFMA A operands: d[0..3] = the 16 code bytes, d[4] = the e8m0
// scale byte. The window of block c = 4j+g starts (sh + c) & 3 = (sh + g) & 3 bytes before
// the block (17 = 1 mod 4), so the byte shift is the same for every step of a lane. Blocks
// past the row end (clamped to the last block, or zero windows) meet an all-zero B operand,
// so any finite operand serves them: their codes are finite whatever the bytes, but their
// scale byte is set to 127, since a misaligned byte could be 0xFF (NaN, and NaN * 0 = NaN).
// Done while the workgroup waits for the gate/up results. N steps from step j0 (the whole
// row, or a part of it where the rows are loaded after the wait).
template <int N = kSteps>
__device__ __forceinline__ void prep_rows(RawBlk (&rw)[N], uint32_t sh, int nb, int g, int j0 = 0) {
  const uint32_t s0 = (sh + (uint32_t)g) & 3u;  // scale byte position
  const uint32_t t = s0 + 1u;                   // code bytes start
  const bool hi = t == 4u;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    RawBlk& r = rw[j];
    const uint32_t sa = 4 * (j0 + j) + g < nb ? (r.d[0] >> (8u * s0)) & 0xFFu : 127u;
    const uint32_t q0 = hi ? r.d[1] : __builtin_amdgcn_alignbyte(r.d[1], r.d[0], t);
    const uint32_t q1 = hi ? r.d[2] : __builtin_amdgcn_alignbyte(r.d[2], r.d[1], t);
    const uint32_t q2 = hi ? r.d[3] : __builtin_amdgcn_alignbyte(r.d[3], r.d[2], t);
    const uint32_t q3 = hi ? r.d[4] : __builtin_amdgcn_alignbyte(r.d[4], r.d[3], t);
    r.d[0] = q0, r.d[1] = q1, r.d[2] = q2, r.d[3] = q3, r.d[4] = sa;
  }
}

// D of one 16-row tile from prepared A operands (prep_rows) and a B image in LDS whose
// blocks from nb up to 4*kSteps-1 and their scale words are zero. Lane (i, g) reads term i&3 (columns
// 4..15 repeat columns 0..3; only columns 0..3 are summed) at fixed offsets from one base:
// block 4j + (g>>1) of step j is at j*512, the block two later at j*512 + 256, and the
// scale byte of block 4j+g at j*16 -- no address arithmetic per step.
// N steps from step j0 accumulate into acc (even steps) and acc1 (odd steps), so a row taken
// in parts gives the same sums as in one pass.
template <int N>
__device__ __forceinline__ void mfma_chain_part(const RawBlk (&rw)[N], const uint8_t* img, const uint32_t* sc,
                                                int i, int g, int j0, f32x4& acc, f32x4& acc1) {
  const uint8_t* bb = img + (g >> 1) * kImgBytes + (i & 3) * 32 + 16 * (g & 1) + j0 * 4 * kImgBytes;
  const uint8_t* sbp = reinterpret_cast<const uint8_t*>(sc) + g * 4 + (i & 3) + j0 * 16;
  // B operands (and scale bytes) of steps j+1 and j+2 are in flight while step j multiplies
  constexpr int kAhead = 2;
  i32x4 b0[kAhead + 1], b1[kAhead + 1];
  int sb[kAhead + 1];
#pragma unroll
  for (int j = 0; j < kAhead; ++j) {
    b0[j] = *reinterpret_cast<const i32x4*>(bb + j * 4 * kImgBytes);
    b1[j] = *reinterpret_cast<const i32x4*>(bb + j * 4 * kImgBytes + 2 * kImgBytes);
    sb[j] = sbp[j * 16];
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int cur = j % (kAhead + 1);
    if (j + kAhead < N) {
      const int nx = (j + kAhead) % (kAhead + 1);
      b0[nx] = *reinterpret_cast<const i32x4*>(bb + (j + kAhead) * 4 * kImgBytes);
      b1[nx] = *reinterpret_cast<const i32x4*>(bb + (j + kAhead) * 4 * kImgBytes + 2 * kImgBytes);
      sb[nx] = sbp[(j + kAhead) * 16];
    }
    __builtin_amdgcn_sched_barrier(0);  // the loads above stay ahead of this step's MFMA
    const i32x8 B = {b0[cur][0], b0[cur][1], b0[cur][2], b0[cur][3], b1[cur][0], b1[cur][1], b1[cur][2], b1[cur][3]};
    const RawBlk& r = rw[j];
    const i32x8 A = {(int)r.d[0], (int)r.d[1], (int)r.d[2], (int)r.d[3], 0, 0, 0, 0};
    if ((j0 + j) & 1)
      acc1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc1, 4, 0, 0, (int)r.d[4], 0, sb[cur]);
    else
      acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc, 4, 0, 0, (int)r.d[4], 0, sb[cur]);
    __builtin_amdgcn_sched_barrier(0);
  }
}
__device__ __forceinline__ f32x4 mfma_chain_p(const RawBlk (&rw)[kSteps], const uint8_t* img,
                                              const uint32_t* sc, int i, int g) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  mfma_chain_part<kSteps>(rw, img, sc, i, g, 0, acc, acc1);
  return f32x4{acc[0] + acc1[0], acc[1] + acc1[1], acc[2] + acc1[2], acc[3] + acc1[3]};
}

// A operands (raw windows) of one 16-row tile, all K steps (S is wave-uniform).
// Blocks past the row end (last step, lane groups g beyond nb) load the row's
// last block instead: their B operand is all zero, so they add exactly 0.
template <int N = kSteps>
__device__ __forceinline__ void issue_rows(const uint8_t* W, int S, int nb, int g, RawBlk (&rw)[N], int j0 = 0) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    if (j0 + j < S)
      raw_load(W + (size_t)min(4 * (j0 + j) + g, nb - 1) * 17, rw[j]);
    else
      raw_zero(rw[j]);
  }
}

// ---- gate/up weight stream -------------------------------------------------------------------
// A wave's 16-row tile (rows adjacent in memory, rb bytes apart) is streamed in chunks of
// kStreamSteps K steps = 4*kStreamSteps blocks: each row's chunk is fetched as kRowPieces
// 16-byte pieces from the 16-byte aligned address at or below its first byte, lane-contiguous,
// so one wave load covers about four rows' contiguous bytes instead of sixteen scattered
// windows. kChunkAhead chunks beyond the one being multiplied are in flight in VGPRs (16 each);
// a landed chunk is written to the wave's LDS buffer (piece index * 16) and the MFMA A windows
// are read back from there (two buffers, alternating). The code is straight-line over the
// kMaxChunks chunks with one uniform branch per chunk, which keeps each chunk's MFMAs next to
// their operands; chunks past the row end load clamped pieces and multiply the zero B line, so
// every path issues the same loads and the compiler's own vmcnt waits stay exact.
constexpr int kStreamSteps = 3;
constexpr int kRowPieces = 15;                    // row slot: 240 bytes
constexpr int kStageLoads = 4;                    // wave loads per chunk (64 pieces each)
constexpr int kStageBytes = kStageLoads * 1024;   // one buffer (pieces past 16 rows land in its pad)
constexpr int kStageOff = 96 * kImgBytes;         // after the largest x image (H <= 3072)
constexpr int kMaxChunks = (kSteps + kStreamSteps - 1) / kStreamSteps;
static_assert(16 * kRowPieces <= kStageLoads * 64, "a chunk's pieces fit one buffer");
static_assert(15 + 17 * 4 * kStreamSteps + 3 <= 16 * kRowPieces, "a row slot holds the chunk and its window tail");
static_assert(kStageOff + 4 * 2 * kStageBytes <= 4 * kImgVec * 1024, "stage buffers fit the dynamic LDS");
static_assert(4 * kSteps * kImgBytes <= kImgVec * 1024 && 4 * kSteps <= 128, "a down slot image holds 4*kSteps blocks");

constexpr int kChunkAhead = 2;  // measured: 1-4 within 1%, 2 best

// Per-lane piece geometry of a 16-row tile, as byte offsets from the tile's first row (W):
// lane piece q = it*64 + lane is piece pc of row `row`; rowa = (W & 15) + row*rb is the row's
// start counted from the 16-byte boundary at or below W, and lastr its last piece.
struct PieceMap {
  uint32_t rowa[kStageLoads], pc16[kStageLoads], lastr[kStageLoads];
};
__device__ __forceinline__ PieceMap piece_map(const uint8_t* W, uint32_t rb, int nb, int lane) {
  PieceMap m;
  const uint32_t a = (uint32_t)(reinterpret_cast<uintptr_t>(W) & 15u);
#pragma unroll
  for (int it = 0; it < kStageLoads; ++it) {
    const int q = it * 64 + lane;
    const int row = min(q / kRowPieces, 15);
    const int pc = min(q - row * kRowPieces, kRowPieces - 1);
    m.rowa[it] = a + (uint32_t)row * rb;
    m.pc16[it] = 16u * (uint32_t)pc;
    m.lastr[it] = (m.rowa[it] + (uint32_t)nb * 17u - 1u) & ~15u;
  }
  return m;
}
// Chunk c of the tile into v (this lane's 4 pieces). Wa = W rounded down to 16 bytes (uniform).
__device__ __forceinline__ void piece_fetch(const uint8_t* Wa, const PieceMap& m, int c, i32x4 (&v)[kStageLoads]) {
  const uint32_t cb = 17u * 4u * kStreamSteps * (uint32_t)c;
#pragma unroll
  for (int it = 0; it < kStageLoads; ++it) {
    const uint32_t first = min((m.rowa[it] + cb) & ~15u, m.lastr[it]);
    const uint32_t off = min(first + m.pc16[it], m.lastr[it]);  // never past the row's last piece
    v[it] = *(const __attribute__((address_space(1))) i32x4*)(Wa + off);  // global, not flat
  }
}

// after_issue() runs once the first chunks' loads are in flight (work that can wait for them).
template <typename F>
__device__ __forceinline__ f32x4 stream_chain_v(const uint8_t* W, uint32_t rb, int nb, uint8_t* stage,
                                                const uint8_t* img, const uint32_t* sc, const uint8_t* zero,
                                                int lane, int i, int g, F&& after_issue) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};  // even / odd steps
  const uint8_t* Wa = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(W) & ~(uintptr_t)15);
  const PieceMap m = piece_map(W, rb, nb, lane);
  const uint32_t rowa_i = (uint32_t)(reinterpret_cast<uintptr_t>(W) & 15u) + (uint32_t)i * rb;  // this lane's row
  const uint32_t last_i = rowa_i + (uint32_t)(nb - 1) * 17u;
  const int nc = (nb + 4 * kStreamSteps - 1) / (4 * kStreamSteps);  // chunks in this row
  i32x4 v[kMaxChunks][kStageLoads];
#pragma unroll
  for (int c = 0; c < kChunkAhead && c < kMaxChunks; ++c) piece_fetch(Wa, m, c, v[c]);
  after_issue();
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    // The branch on c < nc (wave-uniform) also closes a basic block per chunk, which keeps
    // the chunk's MFMAs from being scheduled after later chunks' operand loads.
    if (c >= nc) break;
    // Fetches are unconditional (chunks past the row load clamped pieces), so the loads issued
    // after chunk c are the same on every path and its wait is exact.
    if (c + kChunkAhead < kMaxChunks) piece_fetch(Wa, m, c + kChunkAhead, v[c + kChunkAhead]);
    uint8_t* buf = stage + (c & 1) * kStageBytes;
#pragma unroll
    for (int it = 0; it < kStageLoads; ++it) *reinterpret_cast<i32x4*>(buf + it * 1024 + lane * 16) = v[c][it];
    __builtin_amdgcn_wave_barrier();
    const int b0 = 4 * kStreamSteps * c;
    const int lead = (int)(min(rowa_i + (uint32_t)b0 * 17u, last_i) & 15u);  // chunk start within its first piece
    RawBlk r[kStreamSteps];
    i32x8 B[kStreamSteps];
    int sb[kStreamSteps], off[kStreamSteps];
#pragma unroll
    for (int s = 0; s < kStreamSteps; ++s) {  // every operand of the chunk is loaded first
      const int st = kStreamSteps * c + s;
      const int b = 4 * st + g;
      off[s] = i * (kRowPieces * 16) + lead + (b - b0) * 17;  // <= i*240 + 202: inside the row slot
      const uint32_t* wp = reinterpret_cast<const uint32_t*>(buf + (off[s] & ~3));
      r[s].d[0] = wp[0], r[s].d[1] = wp[1], r[s].d[2] = wp[2], r[s].d[3] = wp[3], r[s].d[4] = wp[4];
      load_b(img, sc, zero, st, nb, i, g, B[s], sb[s]);
    }
#pragma unroll
    for (int s = 0; s < kStreamSteps; ++s) {
      const int st = kStreamSteps * c + s;
      const int b = 4 * st + g;
      if (st & 1)
        acc1 = mfma_raw_nb(r[s], (uint32_t)off[s] & 3u, b < nb, B[s], sb[s], acc1);
      else
        acc = mfma_raw_nb(r[s], (uint32_t)off[s] & 3u, b < nb, B[s], sb[s], acc);
    }
    __builtin_amdgcn_wave_barrier();
  }
  return f32x4{acc[0] + acc1[0], acc[1] + acc1[1], acc[2] + acc1[2], acc[3] + acc1[3]};
}

// ---- the kernel ----------------------------------------------------------------------------
// NORM: the input is rms_norm(x) and the residual x is added to y (mr_moe_forward_residual);
// a separate instantiation, so the plain decode path compiles without that code.
// GEN: a shared expert or more than four slots (top_k + shared). With more than four, the
// down role has one workgroup per row group and group of four slots (a.nsl groups), each
// wave one slot as in the plain case, and the last group of a row group to finish combines
// every slot from the partials buffer. !GEN (top_k <= 4, no shared expert) compiles none of it.
template <bool NORM, bool GEN, bool QWEN>
__global__ __launch_bounds__(256, 3) void k_fused_mxfp4(FusedArgs a) {
  extern __shared__ __align__(16) uint8_t lds_dyn[];
  uint8_t* lds_img = lds_dyn;
  uint32_t* lds_sc = reinterpret_cast<uint32_t*>(lds_dyn + a.lds_img_bytes);
  __shared__ float lds_part[2 * 2 * 2 * 16];  // gate/up: [gate, up][tile][16]; down: [wave][16]
  __shared__ float lds_act[32];
  __shared__ int sel_i[16];
  __shared__ float sel_w[17];  // [k]: weight of the shared expert
  __shared__ int sel_o[16];
  __shared__ uint32_t sel_k[16];
  __shared__ uint32_t route_tmp[128];  // routing: compacted candidates
  __shared__ int ok_flag;
  __shared__ float lds_xw[2];  // gate/up: the shared gate logit and (NORM) the norm scale, as polled
  __shared__ __align__(16) uint8_t lds_zero[32];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int bid = role_index((int)blockIdx.x, a.perm_nc, a.R, a.ND, a.NG);  // role index
  const int nbH = a.H >> 5, nbI = a.I >> 5;
  TRACE(0);
  // This launch's number (wg_seq_word). Its load goes to the device-coherent level, a memory
  // round trip: each role issues it after its own first loads, so that it is in flight with
  // them instead of ahead of them (loaded first, it was waited for before any other load issued).
  uint32_t seq;
  const int has_sh = GEN ? a.has_sh : 0, ktot = GEN ? a.ktot : a.k;
  // Published words: the E logits, the shared expert's gate logit, and with the fused norm its
  // scale 1/sqrt(mean(h^2) + eps), which the gate/up role applies to its dot products instead of
  // reducing the sum of squares itself.
  const uint32_t nlw = (uint32_t)(a.E + has_sh + (NORM ? 1 : 0));
  const RouteCfg rc{a.fs, nlw, a.E, a.k, a.flags, a.wb, a.trace};
  if (tid < 8) reinterpret_cast<uint32_t*>(lds_zero)[tid] = 0u;  // read after later barriers

  if (bid < a.R) {
    // ------------------------------------------------------------- router
    // Logits bid * rr .. bid * rr + rr - 1 (experts, then the shared expert's gate row x . w_gi);
    // wave w takes quarter w of every row's columns, so each wave issues rr * 3 + 3 float4 loads
    // per lane instead of a whole row and x (a CU's address unit takes 64 bytes a clock: loading
    // whole rows kept it busy for most of a microsecond), the quarters' sums are added in quarter
    // order, and wave r finishes logit r.
    __builtin_amdgcn_s_setprio(2);  // the logits gate every other role: router loads issue first
    const int nlog = a.E + has_sh;
    auto router = [&](auto nr_c) {
      constexpr int NR = decltype(nr_c)::value;  // logits of this workgroup
      const int e0 = bid * NR, ef = e0 + wave;    // ef: the logit this wave finishes (wave < NR)
      f32x4 xv[kRouterJ], wv[NR][kRouterJ];      // every load issued before the first use
#pragma unroll
      for (int jj = 0; jj < kRouterJ; ++jj) xv[jj] = ld4_or0(a.x, (lane + 64 * (wave * kRouterJ + jj)) * 4, a.H);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int e = e0 + r;
        // past the last logit (and the shared gate without its input row): x is read instead,
        // a zero logit that is not published
        const float* w = e < a.E ? a.router_w + (size_t)e * a.H : (e == a.E && has_sh) ? a.sh_gate_inp : nullptr;
#pragma unroll
        for (int jj = 0; jj < kRouterJ; ++jj) {
          const int c = (lane + 64 * (wave * kRouterJ + jj)) * 4;
          wv[r][jj] = ld4_or0(w ? w : a.x, w ? c : a.H, a.H);
        }
      }
      // the bias and mask of the logit this wave finishes, loaded with the rows
      const float rbias = (wave < NR && ef < a.E && a.router_b) ? a.router_b[ef] : 0.f;
      const float rmask = (wave < NR && ef < a.E && a.mask) ? a.mask[ef] : 0.f;
      seq = ld_sc1(wg_seq_word(a.fs));
      float inv = 1.f;
      if (NORM) {  // x = rms_norm(h): the quarters' sums of squares, added in quarter order in every wave
        f32x4 nv[kRouterJ];
#pragma unroll
        for (int jj = 0; jj < kRouterJ; ++jj) nv[jj] = ld4_or0(a.nr.w, (lane + 64 * (wave * kRouterJ + jj)) * 4, a.H);
        {
#pragma clang fp contract(off)
          float ss = 0.f;
#pragma unroll
          for (int jj = 0; jj < kRouterJ; ++jj) {
            ss = ss + xv[jj].x * xv[jj].x;
            ss = ss + xv[jj].y * xv[jj].y;
            ss = ss + xv[jj].z * xv[jj].z;
            ss = ss + xv[jj].w * xv[jj].w;
          }
          ss = wave_sum_fast(ss);
          if (lane == 0) lds_part[wave] = ss;
          __syncthreads();
          const float t = ((lds_part[0] + lds_part[1]) + lds_part[2]) + lds_part[3];
          inv = 1.f / sqrtf(t / (float)a.H + a.nr.eps);
        }
#pragma unroll
        for (int jj = 0; jj < kRouterJ; ++jj)
          xv[jj] = f32x4{norm1(xv[jj].x, inv, nv[jj].x), norm1(xv[jj].y, inv, nv[jj].y),
                         norm1(xv[jj].z, inv, nv[jj].z), norm1(xv[jj].w, inv, nv[jj].w)};
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < kRouterJ; ++jj) {
          acc = __builtin_fmaf(xv[jj].x, wv[r][jj].x, acc);
          acc = __builtin_fmaf(xv[jj].y, wv[r][jj].y, acc);
          acc = __builtin_fmaf(xv[jj].z, wv[r][jj].z, acc);
          acc = __builtin_fmaf(xv[jj].w, wv[r][jj].w, acc);
        }
        acc = wave_sum_fast(acc);  // the same bits in every lane
        if (lane == 0) lds_part[16 + r * 4 + wave] = acc;  // (NORM: words 0-3 are not rewritten)
      }
      __syncthreads();
      if (wave < NR && ef < nlog) {
        float acc = ((lds_part[16 + wave * 4] + lds_part[16 + wave * 4 + 1]) + lds_part[16 + wave * 4 + 2]) +
                    lds_part[16 + wave * 4 + 3];
        if (ef < a.E) {
          if (a.router_b) acc = acc + rbias;
          if (a.mask) acc = acc + rmask;
        }
        put_logit(a.fs, nlw, ef, seq, acc);
        if (a.logits_out && ef < a.E && lane == 0) a.logits_out[ef] = acc;
      }
      if (NORM && bid == 0 && wave == 0) put_logit(a.fs, nlw, nlog, seq, inv);  // the norm scale
    };
    if (a.rr == 1) router(std::integral_constant<int, 1>{});
    else if (a.rr == 2) router(std::integral_constant<int, 2>{});
    else router(std::integral_constant<int, kRouterRounds>{});
    TRACE(1);
    prefetch_rows(a.pf, bid, a.R, lds_dyn);
    prefetch_norm(a.pf_nw, a.H, bid, lds_dyn);
  } else if (bid >= a.R + a.ND && bid < a.R + a.ND + a.NG) {
    // ------------------------------------------------------------- gate/up
    const int gid = bid - a.R - a.ND;
    // The gate/up streams issue ahead of the down workgroups' weight prefetch on the same
    // CU (those weights are needed only once every gate/up unit is done).
    __builtin_amdgcn_s_setprio(1);
    const int nrp = a.I >> 5;
    // x split image in LDS (independent of routing): 8 lanes per block, all
    // loads issued first
    {
      constexpr int kRounds = 3;  // 96 blocks / 32 per pass: H <= 3072
      const int m = tid & 7;
      f32x2 lo[kRounds], hi[kRounds];
#pragma unroll
      for (int j = 0; j < kRounds; ++j) {
        const int b = (tid >> 3) + 32 * j;
        const float* xb = a.x + b * 32 + 2 * m;
        if constexpr (NORM) {  // every load issued at once (a clamped block, zero selected after)
          const float* xc = a.x + min(b, nbH - 1) * 32 + 2 * m;
          const f32x2 l0 = *reinterpret_cast<const f32x2*>(xc), h0 = *reinterpret_cast<const f32x2*>(xc + 16);
          lo[j] = b < nbH ? l0 : f32x2{0.f, 0.f};
          hi[j] = b < nbH ? h0 : f32x2{0.f, 0.f};
        } else {  // conditional: fewer requests beside the router's loads (measured faster here)
          lo[j] = b < nbH ? *reinterpret_cast<const f32x2*>(xb) : f32x2{0.f, 0.f};       // 2m, 2m+1
          hi[j] = b < nbH ? *reinterpret_cast<const f32x2*>(xb + 16) : f32x2{0.f, 0.f};  // 2m+16, 2m+17
        }
      }
      if (!NORM) seq = ld_sc1(wg_seq_word(a.fs));
      if (NORM) {  // the image of h * norm_w; the scale 1/rms(h), published by the router, is
                   // applied to the dot products (they are linear in x)
        f32x2 nlo[kRounds], nhi[kRounds];
#pragma unroll
        for (int j = 0; j < kRounds; ++j) {
          const int b = (tid >> 3) + 32 * j;
          const float* wb = a.nr.w + b * 32 + 2 * m;
          nlo[j] = b < nbH ? *reinterpret_cast<const f32x2*>(wb) : f32x2{0.f, 0.f};
          nhi[j] = b < nbH ? *reinterpret_cast<const f32x2*>(wb + 16) : f32x2{0.f, 0.f};
        }
        seq = ld_sc1(wg_seq_word(a.fs));
#pragma unroll
        for (int j = 0; j < kRounds; ++j) {
          lo[j] = f32x2{lo[j].x * nlo[j].x, lo[j].y * nlo[j].y};
          hi[j] = f32x2{hi[j].x * nhi[j].x, hi[j].y * nhi[j].y};
        }
      }
#pragma unroll
      for (int j = 0; j < kRounds; ++j) {
        const int b = (tid >> 3) + 32 * j;
        if (b < nbH) {
          uint32_t codes[kTerms], scales;
          split_block8(lo[j].x, hi[j].x, lo[j].y, hi[j].y, codes, scales);
#pragma unroll
          for (int t = 0; t < kTerms; ++t)
            *reinterpret_cast<uint32_t*>(lds_img + (size_t)b * kImgBytes + t * 32 + 4 * m) = codes[t];
          if (m == 0) lds_sc[b] = scales;
        }
      }
    }
    TRACE(1);
    // The routing wave differs between the (up to four) workgroups that share a CU (dispatch
    // slots b and b + 256 share one), so their polls and selections run on different SIMDs. It
    // alone writes ok_flag: 0 exactly when the selection failed. The selection is finished
    // (weights, order) once its stream is issued.
    RouteState rs;
    const int rw = (int)(blockIdx.x >> 8) & 3;
    if (wave == rw) {
      const bool routed = route_select<MR_ROUTE_SLEEP, QWEN, GEN || NORM>(rc, seq, sel_i, sel_k, route_tmp, rs);
      if (lane == 0) ok_flag = routed ? 1 : 0;
      if (!routed && lane == 0) fail(a.err);
      // the polled extra words: lane 0 the shared gate logit (with a shared expert), the next
      // lane the norm scale (NORM)
      if (GEN && has_sh && lane == 0) lds_xw[0] = rs.xv;
      if (NORM && lane == has_sh) lds_xw[1] = rs.xv;
    }
    XTRACE(wave);  // per wave: at the routing barrier
    __syncthreads();  // selection and x image ready
    TRACE(2);
    if (ok_flag && gid < a.NG) {  // one unit per workgroup
      // units 0 .. k*nrp-1: routed slot unit / nrp; then the shared expert's Ish/32 units
      const int unit = gid, nru = a.k * nrp;
      const bool routed_u = !GEN || unit < nru;  // !GEN: no shared expert, every unit is routed
      const int slot = routed_u ? unit / nrp : a.k, pair = routed_u ? unit % nrp : unit - nru;
      const bool sh = slot >= a.k;  // the shared expert
      const int e = sh ? 0 : sel_i[slot];
      const int tile = wave & 1, mat = wave >> 1;  // mat 0: gate, 1: up
      const int S = (nbH + 3) >> 2;
      const uint64_t rb = (uint64_t)nbH * 17;
      const uint8_t* W = (sh ? (mat ? a.sh_up : a.sh_gate) : expert_at(mat ? a.up : a.gate, e)) +
                         (uint64_t)(pair * 32 + tile * 16) * rb;
      // the epilogue's biases (wave 0, lanes < 32) and shared gate logit, loaded before the stream
      float gbias = 0.f, ubias = 0.f;
      // A logit word reloaded here (agent-coherent, unused without a shared expert) holds back the
      // stream's first wait by a round trip; without it the plain kernel measured 0.15 us slower
      // per launch (the streams then start into the routers' next-layer prefetch and the down
      // workgroups' polls). The shared gate logit itself comes from the routing wave's poll.
      constexpr bool kHold = !NORM;  // with the fused norm the same load made no difference
      const float zhold = kHold ? get_logit(a.fs, nlw, 0) : 0.f;
      if (wave == 0 && lane < 32 && !sh) {
        const size_t bi = (size_t)e * a.I + pair * 32 + lane;
        if (a.gate_b) gbias = a.gate_b[bi];
        if (a.up_b) ubias = a.up_b[bi];
      }
      (void)S;
      f32x4 dacc = stream_chain_v(W, (uint32_t)rb, nbH, lds_img + kStageOff + wave * 2 * kStageBytes, lds_img, lds_sc,
                                  lds_zero, lane, i, g, [&] {
                                    if (wave == rw) route_finish(rc, rs, sel_w, sel_o);
                                  });
      XTRACE(4 + wave);  // per wave: chain done
      TRACE(3);
      if (wave == 0 && has_sh && lane == 0) sel_w[a.k] = a.sh_gate_inp ? sigmoidf_(lds_xw[0] + zhold * 0.f) : 1.f;
      // column sum over the kTerms columns (= quad 0 of each 16-lane row)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float cs = sum4(dacc[r]);
        if (i == 0) lds_part[(mat * 2 + tile) * 16 + 4 * g + r] = cs;
      }
      __syncthreads();
      if (wave == 0) {
        if (lane < 32) {  // rows pair*32 + lane: bias, SwiGLU, routing weight
          const int t2 = lane >> 4, r16 = lane & 15;
          float gv = lds_part[(0 * 2 + t2) * 16 + r16];
          float uv = lds_part[(1 * 2 + t2) * 16 + r16];
          if (NORM) gv = gv * lds_xw[1], uv = uv * lds_xw[1];  // x = (h * norm_w) / rms(h)
          if (!sh && a.gate_b) gv = gv + gbias;
          if (!sh && a.up_b) uv = uv + ubias;
          const float h = (!sh && a.act == MR_ACT_SWIGLU_OAI) ? swiglu_oai(gv, uv, a.alpha, a.limit) : silu_mul(gv, uv);
          lds_act[lane] = h * sel_w[slot];  // written by this wave's route_finish (the shared gate above)
        }
        __builtin_amdgcn_wave_barrier();
        if (lane < 8) {  // split the 32 values: one 32-element block of the down input
          const int m = lane;
          uint32_t codes[kTerms], scales;
          split_block8(lds_act[2 * m], lds_act[2 * m + 16], lds_act[2 * m + 1], lds_act[2 * m + 17],
                       codes, scales);
          const size_t blk = (size_t)slot * nbI + pair;
          uint32_t* dst = reinterpret_cast<uint32_t*>(a.dimg + blk * kImgBytes);
#pragma unroll
          for (int t = 0; t < kTerms; ++t) st_sc1(dst + t * 8 + m, codes[t]);
          if (m == 0) st_sc1(a.dsc + blk, scales);
          vm_drain();  // image stores complete before the count that announces them
        }
      }
      TRACE(4);
    }
    // counted even when routing failed, so later launches stay in step
    if (tid == 0) count<64>(a.fs + FS_GU, gid);
  } else {
    // ------------------------------------------------------------- down
    seq = ld_sc1(wg_seq_word(a.fs));  // needed at once: the routing poll compares its flags
    // Row group q of 16 output rows. The first NS groups are split: rows 0-7 here, rows
    // 8-15 in a workgroup after the gate/up range (half 2). A half's idle lanes read the
    // row of their partner lane (i ^ 8): the same addresses, so no extra HBM bytes.
    // Row group q, slot group sg (slots 4 sg + wave; 0 unless GEN with more than four slots).
    const int tail = bid - (a.R + a.ND + a.NG);
    const int dq = tail >= 0 ? tail : bid - a.R;
    const int q = GEN ? dq % a.NDR : dq, sg = GEN ? dq / a.NDR : 0;
    const int half = tail >= 0 ? 2 : (q < a.NS ? 1 : 0);
    if (tid == 0) ok_flag = 1;
    RouteState rs;  // wave 0: the selection, finished (weights, order) once the prefetch is issued
    // the routing wave runs at the gate/up waves' priority while it selects (its weight
    // prefetch, issued after, stays below the gate/up streams)
    if (wave == 0) __builtin_amdgcn_s_setprio(1);
    if (wave == 0 && !route_select<MR_ROUTE_SLEEP_DOWN, QWEN>(rc, seq, sel_i, sel_k, route_tmp, rs)) {
      if (lane == 0) ok_flag = 0, fail(a.err);
    }
    if (wave == 0) __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    TRACE(1);
    float yres = 0.f, ybias = 0.f;  // this thread's output-row residual and bias terms (tid < 16)
    if (ok_flag) {
      const int row = q * 16 + (half == 0 ? i : (half == 2 ? 8 : 0) + (i & 7));
      RawBlk rd[kSteps];
      const int slot = sg * 4 + wave;  // this wave's slot (routed, then the shared expert)
      const int sl = min(slot, ktot - 1);
      // the slot's K blocks: I/32, or Ish/32 for the shared expert (its image follows the routed
      // slots' images, so slot s's image starts at block s * nbI either way)
      const int nbs = (GEN && sl >= a.k) ? (a.Ish >> 5) : nbI;
      const int S = (nbs + 3) >> 2;
      const uint64_t rb = (uint64_t)nbs * 17;
      const uint8_t* D = (sl >= a.k ? a.sh_down : expert_at(a.down, sel_i[sl])) + (uint64_t)row * rb;
      // the prefetch waits a while: issued at once, its bytes share HBM with the gate/up
      // streams from the start and delay the last gate/up units, which set the hand-off
      for (int it = 0; it < a.dn_delay; ++it) __builtin_amdgcn_s_sleep(8);
      if (slot < ktot) issue_rows(D, S, nbs, g, rd);  // prefetch, independent of gate/up
      if (wave == 0) route_finish(rc, rs, sel_w, sel_o);  // wave 0 alone uses weights and order
      // the combine order in registers (top_k <= 4), so the combine does no dependent LDS reads
      int so[4] = {0, 0, 0, 0};
      if (wave == 0) {
#pragma unroll
        for (int p = 0; p < 4; ++p) so[p] = sel_o[min(p, a.k - 1)] * 16;
      }
      // this thread's output-row bias terms and residual, also independent of gate/up
      if (tid < 16 && NORM && q * 16 + tid < a.H) yres = a.nr.resid[q * 16 + tid];
      if (tid < 16 && a.down_b)
        for (int s2 = 0; s2 < a.k; ++s2) ybias = ybias + sel_w[s2] * a.down_b[(size_t)sel_i[s2] * a.H + q * 16 + tid];
      if (slot < ktot)  // waits for the weights: they land long before gate/up ends
        prep_rows(rd, (uint32_t)reinterpret_cast<uintptr_t>(D) & 3u, nbs, g);
      TRACE(2);
      // polled every 4 sleep units once at most an eighth of the units are missing (+0.3%)
      if (wave == 0 &&
          !wait_count<MR_GU_WAIT_SLEEP, 64, 4>(a.fs + FS_GU, (seq + 1u) * (uint32_t)a.NG, a.wb, (uint32_t)a.NG / 8) &&
          lane == 0)
        ok_flag = 0, fail(a.err);
      __syncthreads();
      TRACE(3);
      if (ok_flag) {
        uint8_t* wimg = lds_img + (size_t)wave * kImgVec * 1024;  // this wave's slot image
        uint32_t* wsc = lds_sc + wave * 128;
        if (slot < ktot) {
          {  // slot image -> LDS with direct global->LDS loads (no VGPRs in flight)
            const uint8_t* src = a.dimg + (size_t)slot * nbI * kImgBytes;
            const int n16 = nbs * kImgBytes / 16;
#pragma unroll
            for (int jj = 0; jj < kImgVec; ++jj) {
              if (64 * jj < n16) {
                const int idx = min(lane + 64 * jj, n16 - 1);
                __builtin_amdgcn_global_load_lds(src + (size_t)idx * 16, wimg + 1024 * jj, 16, 0, 16 /* sc1 */);
              }
            }
            const uint32_t sc0 = ld_sc1(a.dsc + slot * nbI + min(lane, nbs - 1));
            const uint32_t sc1v = ld_sc1(a.dsc + slot * nbI + min(lane + 64, nbs - 1));
            if (lane < nbs) wsc[lane] = sc0;
            if (lane + 64 < nbs) wsc[lane + 64] = sc1v;
            vm_drain();  // the slot image has landed in LDS
            // blocks nbs .. 4*kSteps-1 (read by the last steps, which have all-zero A) and
            // their scale words are zero; after the drain: the last direct load also wrote
            // copies of the final piece there
            for (int z = lane; z < (4 * kSteps - nbs) * (kImgBytes / 16); z += 64)
              reinterpret_cast<i32x4*>(wimg + (size_t)nbs * kImgBytes)[z] = i32x4{0, 0, 0, 0};
            for (int z = nbs + lane; z < 4 * kSteps; z += 64) wsc[z] = 0u;
            __builtin_amdgcn_wave_barrier();
          }
          TRACE(4);
          XTRACE(wave);  // per wave: image in LDS
          const f32x4 d = mfma_chain_p(rd, wimg, wsc, i, g);
          XTRACE(4 + wave);  // per wave: chain done
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float cs = sum4(d[r]);
            if (i == 0) lds_part[wave * 16 + 4 * g + r] = cs;
          }
        }
        __syncthreads();
        if (!GEN || a.nsl == 1) {
          if (tid < 16 && (half == 0 || (tid >> 3) == half - 1)) {
            const int rr = q * 16 + tid;
            float yv = 0.f;  // routed slots in ascending expert order (layer.rs:1092-1106)
#pragma unroll
            for (int p = 0; p < 4; ++p)
              if (p < a.k) yv = yv + lds_part[so[p] + tid];
            yv = yv + ybias;
            if (has_sh) yv = yv + lds_part[a.k * 16 + tid];  // shared expert after the routed sum
            if (NORM) yv = yres + yv;  // hidden = residual + moe_out (layer.rs:473)
            if (rr < a.H) a.y[rr] = yv;
            XTRACE(8);
          }
        } else if (tid < 64 && sg * 4 + (tid >> 4) < ktot) {
          // this slot group's rows -> the partials buffer (combined below)
          st_sc1(reinterpret_cast<uint32_t*>(a.dpart) + (size_t)(sg * 4 + (tid >> 4)) * a.H + q * 16 + (tid & 15),
                 __float_as_uint(lds_part[tid]));
          vm_drain();  // partials complete before the count that announces them
        }
      }
    }
    if (GEN && a.nsl > 1) {
      // The row group's last slot group to finish (a counter per row group, nothing waits)
      // combines every slot. Every slot group counts, also one whose routing or gate/up wait
      // ran out (that launch is reported failed), so the counter stays in step with the launch
      // number for the launches after it.
      __syncthreads();
      if (tid == 0) {
        const bool last = add_sc1(a.fs + FS_DN + q, 1u) + 1u == (seq + 1u) * (uint32_t)a.nsl;
        ok_flag = ok_flag && last ? 2 : 0;
      }
      __syncthreads();
      if (ok_flag == 2 && tid < 16) {
        const int rr = q * 16 + tid;
        const uint32_t* part = reinterpret_cast<const uint32_t*>(a.dpart);
        float yv = 0.f;  // routed slots in ascending expert order (layer.rs:1092-1106)
        for (int p = 0; p < a.k; ++p) yv = yv + __uint_as_float(ld_sc1(part + (size_t)sel_o[p] * a.H + rr));
        yv = yv + ybias;
        if (has_sh) yv = yv + __uint_as_float(ld_sc1(part + (size_t)a.k * a.H + rr));  // shared expert last
        if (NORM) yv = yres + yv;  // hidden = residual + moe_out (layer.rs:473)
        a.y[rr] = yv;
      }
    }
  }
  // ----------------------------------------------------------------- exit
  __syncthreads();
  TRACE(5);
#ifdef MR_FUSED_TRACE
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * 32 + 7] = __smid();
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * 32 + 6] = (unsigned long long)bid + 1;  // role index
  if (a.trace && (threadIdx.x & 63) == 0)  // HW_ID: wave, SIMD, CU, SE of each wave
    a.trace[blockIdx.x * 32 + 26 + (threadIdx.x >> 6)] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
#endif
  if (tid == 0) st_sc1(wg_seq_word(a.fs), seq + 1u);
}

// Shapes the fused kernel runs; others take the VALU path.
// Room for the logits, the shared gate logit and the fused norm's scale.
uint64_t fused_layer_sync_bytes(const mr_layer& L) { return layer_sync_words(L.E + (L.d.sh_gate ? 1u : 0u) + 1u) * 4; }

// More than four slots (top_k > 4, or a shared expert with top_k = 4): one down workgroup
// per row group and group of four slots. A shared expert or more than four slots: the GEN
// instantiation.
static bool fused_multi(const mr_layer& L) { return L.d.top_k + (L.d.sh_gate ? 1u : 0u) > 4u; }
static bool fused_gen(const mr_layer& L) { return L.d.sh_gate != nullptr || fused_multi(L); }

// Logits per router workgroup: the fewest of 1, 2, 4 with which the routers and the down groups
// share one dispatch round (plain layers) or the whole grid fits three workgroups per CU.
static int router_rounds(const mr_layer& L, int n_cu) {
  const uint64_t has_sh = L.d.sh_gate ? 1u : 0u, n = L.E + has_sh, ktot = L.d.top_k + has_sh;
  const uint64_t ND = (L.H + 15) / 16 * ((ktot + 3) / 4), NG = L.d.top_k * (L.I / 32) + has_sh * (L.Ish / 32);
  const bool multi = ktot > 4;
  for (int rr = 1; rr < kRouterRounds; rr *= 2) {
    const uint64_t R = (n + rr - 1) / rr;
    if ((multi || R + ND < (uint64_t)n_cu) && R + ND + NG <= 3ull * n_cu && R + ND + NG <= (uint64_t)kMaxGrid) return rr;
  }
  return kRouterRounds;
}

bool fused_supported(const mr_layer& L, int n_cu) {
  if (L.type != MR_GGML_MXFP4 || L.d.top_k > 16) return false;
  const uint64_t has_sh = L.d.sh_gate ? 1u : 0u;
  if (has_sh && (L.d.sh_gate->type != MR_GGML_MXFP4 || L.d.sh_up->type != MR_GGML_MXFP4 ||
                 L.d.sh_down->type != MR_GGML_MXFP4 || L.Ish % 32 != 0 || L.Ish == 0 ||
                 L.Ish > 32u * 4 * kSteps))
    return false;  // a shared expert: MXFP4 like the routed ones, its K steps within a down wave's
  if (L.E + has_sh > (uint64_t)kMaxLogits) return false;
  const uint64_t ktot = L.d.top_k + has_sh, nsl = (ktot + 3) / 4;
  const uint64_t ND = (L.H + 15) / 16 * nsl, NG = L.d.top_k * (L.I / 32) + has_sh * (L.Ish / 32);
  const uint64_t R = (L.E + has_sh + router_rounds(L, n_cu) - 1) / router_rounds(L, n_cu);
  if (!fused_multi(L) && R + ND >= (uint64_t)n_cu) return false;  // routers and down groups in one dispatch round
  if (R + ND + NG > 3ull * n_cu) return false;
  if (R + ND + NG > (uint64_t)kMaxGrid) return false;  // the split groups are added only where they fit
  const uint64_t nbH = L.H / 32, nbI = L.I / 32;
  if ((nbH + 3) / 4 > (uint64_t)kSteps || (nbI + 3) / 4 > (uint64_t)kSteps) return false;
  if (nbH > 96 || nbI * kImgBytes > (uint64_t)kImgVec * 64 * 16 || nbI > 128) return false;
  if (L.E > 512 || L.H % 32 != 0 || L.I % 32 != 0) return false;
  return true;
}

#ifdef MR_FUSED_TRACE
unsigned long long* g_fused_trace = nullptr;
extern "C" void mr_debug_fused_trace(void* dev_buf) { g_fused_trace = (unsigned long long*)dev_buf; }
#endif

// Grid of a launch: R routers, ND down groups, NG gate/up units and NS split halves.
// Workgroups go to CUs round robin (workgroup b on CU b mod n_cu, three per CU). With
// more than 2 n_cu down and gate/up units, the CUs of the third round that also hold a
// down group carry three units; splitting those down groups in halves, the second half
// in a third-round slot on a CU with two units, caps every CU at 2.5 units.
struct FusedGrid {
  int R, ND, NG, NS, NDR, nsl, rr;
  int total() const { return R + ND + NG + NS; }
};
static FusedGrid fused_grid(const mr_layer& L, int n_cu) {
  FusedGrid g;
  const uint32_t has_sh = L.d.sh_gate ? 1u : 0u, ktot = L.d.top_k + has_sh;
  g.rr = router_rounds(L, n_cu);
  g.R = (int)((L.E + has_sh + g.rr - 1) / g.rr);
  g.NG = (int)(L.d.top_k * (L.I / 32) + has_sh * (L.Ish / 32));
  g.NDR = (int)((L.H + 15) / 16);
  g.nsl = (int)((ktot + 3) / 4);
  g.ND = g.NDR * g.nsl;
  const int grid0 = g.R + g.ND + g.NG;
  g.NS = fused_multi(L) ? 0 : std::max(0, std::min({g.ND + g.NG - 2 * n_cu, g.ND, 3 * n_cu - grid0, kMaxGrid - grid0}));
  return g;
}
// Dynamic LDS of a launch: the gate/up role's x image (nbH blocks), the down role's four
// padded slot images, then the 4-byte scale words.
static uint64_t fused_lds_img_bytes(const mr_layer& L) {
  return std::max<uint64_t>((L.H / 32) * kImgBytes, 4ull * kImgVec * 1024);
}
static uint64_t fused_lds_bytes(const mr_layer& L) {
  return fused_lds_img_bytes(L) + std::max<uint64_t>(L.H / 32, 4ull * 128) * 4;
}

// Every workgroup of a launch must be resident at once (workgroups wait on each other):
// the occupancy the runtime reports for this kernel's registers and LDS, on an otherwise
// idle device, times the CU count must cover the grid (both instantiations).
template <bool NORM>
static const void* fused_kernel(const mr_layer& L) {
  // the near-tie check of probability ranking only where the layer ranks probabilities
  const bool qwen = !(L.d.route_flags & MR_ROUTE_SOFTMAX_AFTER_TOPK);
  if (fused_gen(L))
    return qwen ? reinterpret_cast<const void*>(k_fused_mxfp4<NORM, true, true>)
                : reinterpret_cast<const void*>(k_fused_mxfp4<NORM, true, false>);
  return qwen ? reinterpret_cast<const void*>(k_fused_mxfp4<NORM, false, true>)
              : reinterpret_cast<const void*>(k_fused_mxfp4<NORM, false, false>);
}
bool fused_resident(const mr_layer& L, int n_cu) {
  const size_t lds = fused_lds_bytes(L);
  int b0 = 0, b1 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b0, fused_kernel<false>(L), 256, lds) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&b1, fused_kernel<true>(L), 256, lds) != hipSuccess)
    return false;
  const int grid = fused_grid(L, n_cu).total();
  if ((int64_t)std::min(b0, b1) * n_cu < grid) return false;
  // The occupancy the runtime reports has been seen to count LDS more finely than the CU
  // allocates it (three workgroups of 53.8 KB, reported to fit the 160 KB of a CU, did not all
  // start): a workgroup's LDS, static and dynamic, rounded up to 2 KB, times the workgroups one
  // CU must hold, must fit as well.
  int dev = 0, cu_lds = 0;
  hipFuncAttributes fa{}, fb{};
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cu_lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
      hipFuncGetAttributes(&fa, fused_kernel<false>(L)) != hipSuccess ||
      hipFuncGetAttributes(&fb, fused_kernel<true>(L)) != hipSuccess)
    return false;
  const size_t wg_lds = (std::max(fa.sharedSizeBytes, fb.sharedSizeBytes) + lds + 2047) & ~(size_t)2047;
  return (int64_t)wg_lds * ((grid + n_cu - 1) / n_cu) <= (int64_t)cu_lds;
}

// Delay of the down role's weight prefetch, in s_sleep(8) rounds (512 clocks, about 0.21 us at
// 2.4 GHz): a quarter of the gate/up stream time, estimated from the gate/up bytes at the
// measured stream rate (4.2 TB/s). Swept on C2 (35 MB of gate/up rows) as a fraction of that
// estimate: 0.2 +1.3%, 0.3 and 0.4 +1.8%, 0.5 -4.7% (the down weights then arrive after the
// hand-off). 0.25 stays well below that edge should the shader clock run lower (a lower clock
// lengthens the same number of sleep rounds). Plain layers only (top-k <= 4, no shared
// expert), where it was measured.
static int dn_delay_rounds(const mr_layer& L) {
  if (fused_gen(L)) return 0;
  const double gu_bytes = 2.0 * (double)L.d.top_k * (double)L.I * (double)(L.H / 32) * 17.0;
  return (int)(0.25 * gu_bytes / 4.2e6 / 0.213 + 0.5);
}

hipError_t launch_fused(const Launch& K, const mr_layer& L, const float* x, float* y,
                        uint32_t* err, uint8_t* img_base, WaitBound wb, int n_cu,
                        const NormResid& nr) {
  FusedArgs a{};
#ifdef MR_FUSED_TRACE
  a.trace = g_fused_trace;
#endif
  a.gate = expert_loc(L.d.gate), a.up = expert_loc(L.d.up), a.down = expert_loc(L.d.down);
  a.gate_b = L.d.gate_bias, a.up_b = L.d.up_bias, a.down_b = L.d.down_bias;
  a.router_w = L.d.router_w, a.router_b = L.d.router_b, a.mask = L.d.dummy_mask;
  a.has_sh = L.d.sh_gate ? 1 : 0;
  if (a.has_sh) {
    a.sh_gate = L.d.sh_gate->base + L.d.sh_gate->h_offsets[0];
    a.sh_up = L.d.sh_up->base + L.d.sh_up->h_offsets[0];
    a.sh_down = L.d.sh_down->base + L.d.sh_down->h_offsets[0];
    a.sh_gate_inp = L.d.sh_gate_inp;
  }
  a.x = x, a.y = y, a.fs = L.fused_sync, a.err = err;
  a.logits_out = L.logits_out;
  const uint64_t nbH = L.H / 32, nbI = L.I / 32, k = L.d.top_k, ktot = k + (uint64_t)a.has_sh;
  a.dimg = img_base;
  const uint64_t nblk = k * nbI + (a.has_sh ? L.Ish / 32 : 0);  // image blocks of every slot
  a.dsc = reinterpret_cast<uint32_t*>(img_base + nblk * kImgBytes);
  a.dpart = reinterpret_cast<float*>(img_base + ((nblk * (kImgBytes + 4) + 255) & ~(uint64_t)255));
  a.Ish = a.has_sh ? (int)L.Ish : 0;
  a.H = (int)L.H, a.I = (int)L.I, a.E = (int)L.E, a.k = (int)k, a.ktot = (int)ktot;
  a.flags = L.d.route_flags, a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  const FusedGrid fg = fused_grid(L, n_cu);
  a.R = fg.R, a.NG = fg.NG, a.ND = fg.ND, a.NS = fg.NS, a.NDR = fg.NDR, a.nsl = fg.nsl, a.rr = fg.rr;
  a.perm_nc = role_perm_nc(fg.total(), fg.R, fg.NG, n_cu);
  a.dn_delay = dn_delay_rounds(L);
  a.wb = wb;
  a.pf = prefetch_plan(L.next);
  if (a.pf.w && L.next->type == MR_GGML_MXFP4 && L.next->ctx) a.pf.rpw = router_rounds(*L.next, n_cu);
  a.pf_nw = L.next && L.next->H == L.H ? L.next->norm_w : nullptr;
  a.nr = nr;
  a.lds_img_bytes = (uint32_t)fused_lds_img_bytes(L);
  const size_t lds = fused_lds_bytes(L);
  (void)nbH;
  ProfScope ps(K, "fused_layer");
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel(nr.w ? fused_kernel<true>(L) : fused_kernel<false>(L), dim3(fg.total()), dim3(256),
                                       args, lds, K.s);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace mr
