// mr_grouped.hip -- multi-token (prefill / batched) MXFP4 MoE experts as grouped
// GEMMs on the gfx950 scaled MX-fp4 MFMA.
//
// The reference runs each expert once over all of its tokens: index_select of
// the expert's tokens, gate/up/act/down, x routing weight, index_add back
// (layer.rs:2148-2183; CPU: mxfp4_matmul per expert, layer.rs:1449-1514). Here:
//   k_group       (token, slot) pairs grouped by expert; per-expert pair offsets and
//                 32-pair tile offsets; pair index of every (token, slot).
//   k_split_rows  x rows -> e4m3 B images (terms 0-2 of the split of each 32-element block).
//   k_grouped_gemm<true>   gate and up for one (expert, 128-row tile, 32-pair tile):
//                 A = native MXFP4 weight rows, B = the pairs' x images; epilogue
//                 bias + activation x routing weight, split into the h images
//                 [pair][I/32] (the split of k_split_rows).
//   k_grouped_gemm<false>  down for one (expert, 256-row tile, 32-pair tile) on the
//                 h images -> o [pair][H].
//   k_combine     y[t] = sum over t's pairs in ascending expert order of
//                 (o + w*b_down) (the order of layer.rs:1092-1106).
// Every weight byte of an expert is read by the ceil(n_e/32) pair tiles of its
// row tiles; work items are laid out so those repeats, and the repeats of the
// pairs' activation images over row tiles, hit the same XCD's L2.
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"
#include "mr_mx_mfma.h"

#include <algorithm>
#include <climits>
#include <type_traits>

namespace mr {

// Terms of the activation split that the grouped GEMMs read, and all that their splits
// compute and write (the images keep the 4-term layout; term 3 is left unwritten).
constexpr int kGemmTerms = 3;

constexpr int kPairTile = 32;   // pairs (tokens) per work item = 8 MFMA column groups x 4
constexpr int kXcds = 8;        // MI355X accelerator complex dies (one L2 each)
constexpr int kMaxSteps = 32;   // K steps (4 blocks) per row: K <= 4096

// ---- grouping ---------------------------------------------------------------------------
// One workgroup: count the (token, slot) entries of every expert, lay the experts out in
// order (exp_off, tile_off), and give every entry a position inside its expert's range by
// an LDS counter. The order of the entries inside an expert depends on timing, but nothing
// computed from them does: each pair's GEMM column and epilogue depend on that pair alone,
// and a token's pairs are combined in ascending expert order, which the ranges fix.
__global__ __launch_bounds__(256) void k_group(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                               int P, int k, int E, int32_t* __restrict__ pair_tok,
                                               float* __restrict__ pair_w, int32_t* __restrict__ pair_of,
                                               int32_t* __restrict__ exp_off, int32_t* __restrict__ tile_off) {
  __shared__ int cnt[1024];
  const int tid = threadIdx.x, lane = tid & 63;
  for (int e = tid; e < E; e += 256) cnt[e] = 0;
  __syncthreads();
  constexpr int kGJ = 8;  // entries per thread whose loads are issued together (one round trip)
  const bool one = P <= 256 * kGJ;  // one pass: the entries and weights stay in registers
  int ev[kGJ];
  float wv[kGJ];
  for (int b0 = 0; b0 < P; b0 += 256 * kGJ) {
#pragma unroll
    for (int j = 0; j < kGJ; ++j) {
      const int q = b0 + 256 * j + tid;
      ev[j] = q < P ? min(max(idx[q], 0), E - 1) : -1;
      wv[j] = (one && q < P) ? w[q] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kGJ; ++j)
      if (ev[j] >= 0) atomicAdd(&cnt[ev[j]], 1);
  }
  __syncthreads();
  if (tid < 64) {  // expert offsets, in expert order: lane l takes experts 16l .. 16l+15 (E <= 1024)
    int c[16], s = 0, ts = 0;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = 16 * lane + u;
      c[u] = e < E ? cnt[e] : 0;
      s += c[u], ts += (c[u] + kPairTile - 1) / kPairTile;
    }
    int po = s, to = ts;  // inclusive prefix over lanes, then exclusive
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(po, o, 64), b = __shfl_up(to, o, 64);
      if (lane >= o) po += a, to += b;
    }
    po -= s, to -= ts;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = 16 * lane + u;
      if (e < E) {
        exp_off[e] = po, tile_off[e] = to;
        cnt[e] = po;  // becomes the next free position
      }
      po += c[u], to += (c[u] + kPairTile - 1) / kPairTile;
    }
    if (16 * lane < E && E <= 16 * lane + 16) exp_off[E] = po, tile_off[E] = to;
  }
  __syncthreads();
  for (int b0 = 0; b0 < P; b0 += 256 * kGJ) {
    if (!one) {
#pragma unroll
      for (int j = 0; j < kGJ; ++j) {
        const int q = b0 + 256 * j + tid;
        ev[j] = q < P ? min(max(idx[q], 0), E - 1) : -1;
        wv[j] = q < P ? w[q] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < kGJ; ++j) {
      if (ev[j] >= 0) {
        const int q = b0 + 256 * j + tid;
        const int pos = atomicAdd(&cnt[ev[j]], 1);
        pair_tok[pos] = q / k, pair_w[pos] = wv[j], pair_of[q] = pos;
      }
    }
  }
}

// ---- activation rows -> B images ------------------------------------------------------------
// Row r of `src` (D floats) -> img[r][D/32][kImgBytes] + sc[r][D/32]; 8 lanes per block, on a
// (block groups of 32, rows) grid (rows past gridDim.y loop).
__global__ __launch_bounds__(256) void k_split_rows(const float* __restrict__ src, int n_rows, int D,
                                                    uint8_t* __restrict__ img, uint32_t* __restrict__ sc) {
  const int nb = D >> 5;
  const int b = blockIdx.x * 32 + (threadIdx.x >> 3);
  const int m = threadIdx.x & 7;
  const bool in = b < nb;  // the same for the block's 8 lanes (the split's DPP stays in them)
  for (int r = blockIdx.y; r < n_rows; r += gridDim.y) {
    const float* p = src + (size_t)r * D + min(b, nb - 1) * 32 + 2 * m;
    const f32x2 lo = *reinterpret_cast<const f32x2*>(p);       // elements 2m, 2m+1
    const f32x2 hi = *reinterpret_cast<const f32x2*>(p + 16);  // elements 2m+16, 2m+17
    uint32_t codes[kTerms], scales;
    split_block8<kGemmTerms>(lo.x, hi.x, lo.y, hi.y, codes, scales);
    if (in) {
      const size_t bb = (size_t)r * nb + b;
      uint32_t* dst = reinterpret_cast<uint32_t*>(img + bb * kImgBytes);
#pragma unroll
      for (int t = 0; t < kGemmTerms; ++t) dst[t * 8 + m] = codes[t];
      if (m == 0) sc[bb] = scales;
    }
  }
}

// ---- grouped GEMM -------------------------------------------------------------------------
struct GroupedArgs {
  ExpertLoc w0;  // gate (GATEUP) or down
  ExpertLoc w1;  // up (GATEUP)
  const float* b0;  // gate bias [E][M] (GATEUP) or null
  const float* b1;  // up bias
  const uint8_t* img;    // B images [rows][K/32][kImgBytes]
  const uint32_t* isc;   // [rows][K/32]
  const int32_t* pair_tok;  // B row of pair p (GATEUP: its token) or null (row = p)
  const float* pair_w;      // GATEUP: routing weight of pair p, or null (weight 1)
  const int32_t* exp_off;
  const int32_t* tile_off;
  int single_p;  // > 0: one expert (e = 0) over pairs 0 .. single_p - 1 (the shared expert over
                 // every token); exp_off and tile_off are not read
  float* out;        // [P][M] (down)
  uint8_t* himg;     // GATEUP: the down input images [P][M/32][kImgBytes]
  uint32_t* hsc;     // GATEUP: their scale words [P][M/32]
  int M, K, E;
  int act;
  float alpha, limit;
};

// Grouped GEMM work item: (expert e, row tile, 32-pair tile); 4 waves. A wave owns kGT
// 16-row A tiles (gate/up: 32 gate rows and the same 32 up rows, so that the activation and the
// split of the down input image run in registers, 128 rows per item; down: 4 x 64 = 256 rows)
// and the tile's 32 pairs as 2 groups of 16.
// The MFMAs take the first kGemmTerms = 3 e4m3 terms of the pairs' activation split (the
// residual after three terms is below 2^-12 of each 32-element block's max, bf16 operands
// hold 8 significant bits). A K step holds 4 weight blocks; MFMA m of the step takes term m of
// all four: K block j of MFMA m is weight block j (its A operand: native MXFP4 codes and the
// block's scale byte, read per lane) against term m of block j of the 16 pairs (with that
// term's scale byte). A lane's A operand is then the same in the step's 3 MFMAs, so each A
// window is read from LDS and aligned once per step, and D accumulates the term-summed dot
// product of row x pair: no term columns to add afterwards, 16 pairs per MFMA, and a wave
// keeps kGT x 2 accumulator tiles.
// K advances 4 blocks per step:
//   A: each row's 68 bytes of a step as 6 aligned 16-byte pieces, lane-contiguous (a wave
//      load covers ~11 rows' contiguous bytes; 20-byte windows loaded per lane straight
//      from global cost 3x the L1 accesses), two steps ahead in registers, then written to
//      the wave's LDS slice, from which the 4 lanes of a row read the same block window;
//   B: the step's 32 pairs x 4 blocks x the 96 bytes of terms 0-2 of their images (12 KB) and
//      their scale words, one step ahead in registers (3 pieces per thread; the images are L2
//      hits), then written to a double-buffered LDS stage shared by the 4 waves. (Direct global->LDS loads would save the registers, but
//      the compiler then waits for all of them before any LDS read, which serialises the
//      prefetch.) 16-byte part q of (pair pr, block b) sits in slot b_slot(pr, b, q),
//      so the 16 lanes of a read (16 pairs, one part) hit 16 different bank groups.
constexpr int kGW = 4;               // waves per work item
#ifndef MR_GROUPED_GT_GU
#define MR_GROUPED_GT_GU 4
#endif
#ifndef MR_GROUPED_GT_DN
#define MR_GROUPED_GT_DN 4
#endif
// 16-row A tiles per wave (gate/up, down) and the rows of a matrix per work item
template <bool GATEUP> constexpr int kGTof = GATEUP ? MR_GROUPED_GT_GU : MR_GROUPED_GT_DN;
template <bool GATEUP> constexpr int kRowsOf = (GATEUP ? kGW / 2 : kGW) * kGTof<GATEUP> * 16;
constexpr int kPG = kPairTile / 16;  // 16-pair MFMA column groups
constexpr int kBStep = kPairTile * 4 * kImgBytes;  // B bytes per K step
constexpr int kAPR = 6;                            // A pieces per row and step: 68 bytes at any offset
#ifndef MR_GROUPED_AROW
#define MR_GROUPED_AROW 104
#endif
constexpr int kARow = MR_GROUPED_AROW;  // LDS bytes per A row: 26 dwords, so 16 rows fall in 16 different banks
static_assert(kARow % 4 == 0 && kARow >= 6 * 16, "an A row holds a step's 6 pieces, dword-aligned");
constexpr int kBBuf = 2;                           // B stages in LDS
static_assert(kBStep == 4 * kGW * 64 * 16, "room for four 16-byte pieces per thread per step");
constexpr int kBPieces = 3;  // 16-byte B pieces loaded per thread and step (terms 0-2)
static_assert(kPairTile * 4 * 6 == kBPieces * kGW * 64, "the pieces of terms 0-2 fill the threads");
static_assert(kPairTile * 4 == 2 * 64, "scale words: one per lane of waves 0-1");
static_assert(kTerms == 4, "images of 4 terms (8 parts of 16 bytes per block); the GEMMs read terms 0-2");

// LDS slot of 16-byte part q of (pair pr, block b) in a B stage: the 16 pairs that one read
// instruction's lanes take (one part each) land in 16 different 16-byte bank groups.
__device__ __forceinline__ int b_slot(int pr, int b, int q) { return pr * 32 + (b ^ ((pr >> 3) & 1)) * 8 + (q ^ (pr & 7)); }

template <bool GATEUP>
__global__ __launch_bounds__(256, 2) void k_grouped_gemm(GroupedArgs a) {
  __shared__ __align__(16) uint8_t bst[kBBuf][kBStep];
  __shared__ __align__(16) uint32_t bsc[kBBuf][kPairTile * 4];
  constexpr int kGT = kGTof<GATEUP>;               // 16-row A tiles per wave
  constexpr int kASlots = kGT * 16 * kAPR;         // A pieces per wave and step
  constexpr int kAK = (kASlots + 63) / 64;         // A piece loads per lane and step
  __shared__ __align__(16) uint8_t ast[kGW][kGT * 16 * kARow];
  __shared__ float bias_s[GATEUP ? 2 * (kGW / 2) * kGT * 16 + kPairTile : 1];  // GATEUP: the tile's gate,
                                                                               // up biases, pair weights
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: wave-level branches stay scalar
  const int i = lane & 15, g = lane >> 4;
  constexpr int kRows = kRowsOf<GATEUP>;  // rows of a matrix per item
  // Work items are ordered (expert, row tile, pair tile of the expert), and each XCD
  // (workgroups are dispatched round-robin over kXcds) takes one contiguous range of them:
  // the items that share an expert's row tile (A) or its pairs' images (B) run on the same
  // XCD and meet in its L2.
  const int n_rt = (a.M + kRows - 1) / kRows;
  const bool single = a.single_p > 0;
  const int n_tiles = single ? (a.single_p + kPairTile - 1) / kPairTile : a.tile_off[a.E];
  const int n_work = n_rt * n_tiles;
  const int per_xcd = (n_work + kXcds - 1) / kXcds;
  const int loc = blockIdx.x / kXcds;
  const int w = (blockIdx.x % kXcds) * per_xcd + loc;
  if (loc >= per_xcd || w >= n_work) return;  // uniform: no work item for this workgroup
  int lo = 0, hi = single ? 1 : a.E;  // expert: n_rt * tile_off[e] <= w < n_rt * tile_off[e+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (n_rt * a.tile_off[mid] <= w) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int e_beg = single ? 0 : a.exp_off[e], e_end = single ? a.single_p : a.exp_off[e + 1];
  const int nt_e = single ? n_tiles : a.tile_off[e + 1] - a.tile_off[e];
  const int wl = w - (single ? 0 : n_rt * a.tile_off[e]);
  const int rt = wl / nt_e, tl = wl - rt * nt_e;
  const int p0 = e_beg + tl * kPairTile;
  const int np = min(kPairTile, e_end - p0);
  const int npg = (np + 15) >> 4;  // pair groups holding pairs (uniform)

  const int nbK = a.K >> 5, S = (nbK + 3) >> 2;
  const uint64_t rb = (uint64_t)nbK * 17;
  // Rows of this wave: gate/up: tiles 0 .. kTR-1 are the gate rows wrow0 .. wrow0 + 16 kTR - 1
  // and tiles kTR .. 2kTR-1 the same up rows, so that a lane holds the gate and up values of
  // the same (row, pair) for the activation; down: kGT tiles of consecutive rows.
  constexpr int kTR = GATEUP ? kGT / 2 : kGT;  // 16-row tiles per matrix of a wave
  static_assert(!GATEUP || kGT == 4, "gate/up: two gate and two up tiles, one 32-row split block per wave");
  const int wrow0 = rt * kRows + wave * (kTR * 16);
  if (GATEUP) {  // read by the epilogue (after the K loop's barriers)
    for (int q = tid; q < 2 * kRows + kPairTile; q += kGW * 64) {
      if (q < 2 * kRows) {
        const int mat = q >= kRows, orow = rt * kRows + q - mat * kRows;
        const float* bsrc = mat ? a.b1 : a.b0;
        bias_s[q] = (bsrc && orow < a.M) ? bsrc[(size_t)e * a.M + orow] : 0.f;
      } else {
        bias_s[q] = a.pair_w ? a.pair_w[p0 + min(q - 2 * kRows, np - 1)] : 1.f;
      }
    }
  }
  const uint8_t* Wm[2] = {expert_at(a.w0, e), GATEUP ? expert_at(a.w1, e) : expert_at(a.w0, e)};
  // This lane's row i: its rows in every tile of one matrix are 16 rows (a multiple of 16
  // bytes) apart, so the byte position of a block in its 16-byte piece is the same for all of
  // them (lead0[matrix]; the gate and up matrices may start at different offsets).
  uint32_t lead0[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
    lead0[mt] = (uint32_t)(reinterpret_cast<uintptr_t>(Wm[mt]) + (uintptr_t)min(wrow0 + i, a.M - 1) * rb) & 15u;
  // A piece slots of this lane: slot k*64 + lane = (tile, row, piece) of the wave's rows
  const uint8_t* aps[kAK];
  int apc[kAK], aslot[kAK];
#pragma unroll
  for (int k = 0; k < kAK; ++k) {
    const int sl = min(k * 64 + lane, kASlots - 1);
    const int tt = sl / (16 * kAPR), rr = (sl / kAPR) % 16;
    apc[k] = sl % kAPR;
    aps[k] = Wm[tt / kTR] + (uint64_t)min(wrow0 + 16 * (tt % kTR) + rr, a.M - 1) * rb;
    aslot[k] = (tt * 16 + rr) * kARow + apc[k] * 16;
  }

  // B pieces of this thread: the step's 32 pairs x 4 blocks x the 6 16-byte parts of terms
  // 0-2 (term 3 is not used) are 768 pieces, 3 per thread: piece j*256 + tid = (pair, block,
  // part) in that order, so consecutive lanes read consecutive parts of a block
  const uint8_t* bsrc[kBPieces];
  int bslot[kBPieces], bblk[kBPieces];
#pragma unroll
  for (int j = 0; j < kBPieces; ++j) {
    const int q = j * 256 + tid, part = q % 6, blk = (q / 6) & 3, pr = q / 24;
    bslot[j] = b_slot(pr, blk, part);
    bblk[j] = blk;
    const int p = p0 + min(pr, np - 1);
    const int r = a.pair_tok ? a.pair_tok[p] : p;
    bsrc[j] = a.img + (size_t)r * nbK * kImgBytes + part * 16;
  }
  const uint32_t* ssrc;  // scale word tid (waves 0-1): pair tid/4, block tid%4
  {
    const int p = p0 + min((tid & 127) >> 2, np - 1);
    const int r = a.pair_tok ? a.pair_tok[p] : p;
    ssrc = a.isc + (size_t)r * nbK;
  }
  struct BRegs {
    i32x4 v[kBPieces];
    uint32_t sc;
  };
  auto load_b = [&](int st, BRegs& br) {
#pragma unroll
    for (int j = 0; j < kBPieces; ++j) {
      const size_t boff = (size_t)min(4 * st + bblk[j], nbK - 1) * kImgBytes;
      br.v[j] = *(const __attribute__((address_space(1))) i32x4*)(bsrc[j] + boff);
    }
    br.sc = *(const __attribute__((address_space(1))) uint32_t*)(ssrc + min(4 * st + (tid & 3), nbK - 1));
  };
  auto store_b = [&](const BRegs& br, int buf) {
#pragma unroll
    for (int j = 0; j < kBPieces; ++j) *reinterpret_cast<i32x4*>(&bst[buf][bslot[j] * 16]) = br.v[j];
    if (wave < 2) bsc[buf][tid] = br.sc;
  };
  auto load_a = [&](int st, i32x4 (&apv)[kAK]) {  // pieces past the row end read its last piece
#pragma unroll
    for (int k = 0; k < kAK; ++k) {
      const uintptr_t first = (reinterpret_cast<uintptr_t>(aps[k]) + (uintptr_t)(68 * st)) & ~(uintptr_t)15;
      const uintptr_t last = (reinterpret_cast<uintptr_t>(aps[k]) + (uintptr_t)(17 * nbK) - 1) & ~(uintptr_t)15;
      const uintptr_t src = min(first + 16 * (uintptr_t)apc[k], last);
      apv[k] = *(const __attribute__((address_space(1))) i32x4*)src;
    }
  };
  auto store_a = [&](const i32x4 (&apv)[kAK]) {  // slots past kASlots are not stored
#pragma unroll
    for (int k = 0; k < kAK; ++k)
      if (k * 64 + 64 <= kASlots || k * 64 + lane < kASlots)
        {
          if constexpr (kARow % 8 == 0) {  // 8-byte aligned: rows are kARow bytes apart
            uint64_t* d = reinterpret_cast<uint64_t*>(&ast[wave][aslot[k]]);
            d[0] = ((uint64_t)(uint32_t)apv[k][1] << 32) | (uint32_t)apv[k][0];
            d[1] = ((uint64_t)(uint32_t)apv[k][3] << 32) | (uint32_t)apv[k][2];
          } else {
            uint32_t* d = reinterpret_cast<uint32_t*>(&ast[wave][aslot[k]]);
            d[0] = (uint32_t)apv[k][0], d[1] = (uint32_t)apv[k][1], d[2] = (uint32_t)apv[k][2], d[3] = (uint32_t)apv[k][3];
          }
        }
  };
  // MFMA m of a step takes term m of the activation split for all 4 blocks of the step. Lane
  // (pair i of the group, K group g): its A operand is weight block g of the step in all three
  // MFMAs; its B bytes 0-15 are K [16g, 16g+16), half g%2 of K block g/2, and bytes 16-31 half
  // g%2 of K block 2 + g/2, i.e. part 2m + g%2 of (pair i, block g/2) and of (pair i, block
  // 2 + g/2), which b_slot places 16 slots (256 bytes) further; its B scale byte is (pair i,
  // block g, term m) at 16i + 4g + m. Pairs of the two groups differ by 16 (the same swizzle;
  // scale bytes +256). brdp holds the slot of MFMA m's first part in bits 10m .. 10m + 9.
  uint32_t brdp = 0u;
#pragma unroll
  for (int mm = 0; mm < 3; ++mm) brdp |= (uint32_t)b_slot(i, g >> 1, 2 * mm + (g & 1)) << (10 * mm);
  const int sc_lane = i * 16 + 4 * g;
  auto brd = [&](int mm) { return (int)(__builtin_amdgcn_ubfe(brdp, 10u * (uint32_t)mm, 10u) * 16u); };

  i32x4 apA[kAK], apB[kAK];
  BRegs bR;
  load_b(0, bR);
  load_a(0, apA);
  load_a(min(1, S - 1), apB);

  f32x4 acc[kGT][kPG];
#pragma unroll
  for (int tt = 0; tt < kGT; ++tt)
#pragma unroll
    for (int pg = 0; pg < kPG; ++pg) acc[tt][pg] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step st: A pieces in register set st % 2 (loaded two steps ahead), B pieces in one
  // register set (one step ahead: the images are L2 hits), B in LDS buffer st % 2. Every step
  // issues the same loads, B first (past the last step: the last step's data again), so the
  // compiler's waits before the LDS writes count exactly the loads issued after them.
  // `part` (a std::bool_constant): the step may hold blocks past the row end. Only such steps
  // test every A window for it; full steps compile without those selects.
  auto step = [&](int st, i32x4 (&cur)[kAK], auto part) {
    constexpr bool kPart = decltype(part)::value;
    const int buf = st % kBBuf;
    store_a(cur);      // this wave's A slice (its reads of step st-1 are done: LDS ops stay in order)
    store_b(bR, buf);  // buffer st % 2 was last read in step st-2, before the previous barrier
    __syncthreads();   // step st's B stage is complete
    load_b(min(st + 1, S - 1), bR);
    load_a(min(st + 2, S - 1), cur);
    const uint8_t* bb_base = &bst[buf][0];
    const uint8_t* sc_base = reinterpret_cast<const uint8_t*>(&bsc[buf][0]);
    uint32_t wo[2];  // per matrix: block g's scale byte in the row's LDS slice (68 st = 4 st mod 16)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) wo[mt] = ((lead0[mt] + 4u * (uint32_t)st) & 15u) + 17u * (uint32_t)g;
    // B operands of MFMA mm for the 2 pair groups, read one MFMA ahead; the A operands (this
    // lane's block g of each tile's row i) once per step for all three MFMAs. A block past the
    // row end (read inside the LDS stage) gets zero codes, so it adds nothing.
    struct BOps {
      i32x4 b[kPG][2];
      int sb[kPG];
    };
    auto read_b = [&](int mm, BOps& o) {
      const int off = brd(mm);
#pragma unroll
      for (int pg = 0; pg < kPG; ++pg) {
        const uint8_t* bp = bb_base + pg * 16 * 32 * 16 + off;  // pairs 16 further: same swizzle
        o.b[pg][0] = *reinterpret_cast<const i32x4*>(bp);
        o.b[pg][1] = *reinterpret_cast<const i32x4*>(bp + 256);
        o.sb[pg] = (int)sc_base[sc_lane + mm + pg * 256];
      }
    };
    RawBlk r[kGT];
#pragma unroll
    for (int tt = 0; tt < kGT; ++tt) {
      const uint32_t* wp = reinterpret_cast<const uint32_t*>(&ast[wave][(tt * 16 + i) * kARow + (wo[tt / kTR] & ~3u)]);
      r[tt].d[0] = wp[0], r[tt].d[1] = wp[1], r[tt].d[2] = wp[2], r[tt].d[3] = wp[3], r[tt].d[4] = wp[4];
    }
    BOps o0, o1;
    read_b(0, o0);
    read_b(1, o1);
    const bool valid = !kPart || 4 * st + g < nbK;
    AOp ao[kGT];
    int sa[kGT];
#pragma unroll
    for (int tt = 0; tt < kGT; ++tt) {
      // byte alignment by v_alignbyte (a shift of 4 bytes selects the upper dword): the same
      // as shifting the dword pair right by t bytes, which the compiler would otherwise do
      // through a stack copy of the window
      const uint32_t w3 = wo[tt / kTR] & 3u, t = w3 + 1u;  // the codes start t bytes into the window (1..4)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t v = t == 4u ? r[tt].d[q + 1] : __builtin_amdgcn_alignbyte(r[tt].d[q + 1], r[tt].d[q], t);
        ao[tt].q[q] = valid ? v : 0u;
      }
      sa[tt] = valid ? (int)((r[tt].d[0] >> (8u * w3)) & 0xFFu) : 127;
    }
    auto run_b = [&](const BOps& o) {
#pragma unroll
      for (int pg = 0; pg < kPG; ++pg) {
        if (pg < npg) {
          const i32x8 B = {o.b[pg][0][0], o.b[pg][0][1], o.b[pg][0][2], o.b[pg][0][3],
                           o.b[pg][1][0], o.b[pg][1][1], o.b[pg][1][2], o.b[pg][1][3]};
#pragma unroll
          for (int tt = 0; tt < kGT; ++tt)  // tiles past M repeat row M-1; their rows are not stored
            acc[tt][pg] = mfma_op(ao[tt], sa[tt], B, o.sb[pg], acc[tt][pg]);
        }
      }
    };
    run_b(o0);
    read_b(2, o0);
    run_b(o1);
    run_b(o0);
  };
  // Steps 0 .. nbK/4 - 1 hold only blocks inside the row; the one or two steps after the loop
  // (the last one possibly partial) run the checked variant.
  const int s_full = nbK >> 2;
  int st = 0;
  for (; st + 1 < s_full; st += 2) {
    step(st, apA, std::false_type{});
    step(st + 1, apB, std::false_type{});
  }
  if (st < S) {
    step(st, apA, std::true_type{});
    if (st + 1 < S) step(st + 1, apB, std::true_type{});
  }

  // Epilogue: acc[tt][pg][r] of lane (i, g) is row wrow0 + 16 tt + 4g + r x pair 16 pg + i.
  if constexpr (!GATEUP) {  // down: the lane's 4 consecutive rows of a pair as one 16-byte store
#pragma unroll
    for (int tt = 0; tt < kGT; ++tt)
#pragma unroll
      for (int pg = 0; pg < kPG; ++pg) {
        const int pl = pg * 16 + i, row = wrow0 + 16 * tt + 4 * g;  // M % 32 == 0: row < M -> row + 3 < M
        if (pl < np && row < a.M) *reinterpret_cast<f32x4*>(a.out + (size_t)(p0 + pl) * a.M + row) = acc[tt][pg];
      }
    return;
  }
  // Gate/up: lane (i, g) holds gate rows 4g .. 4g+3 and 16+4g .. 16+4g+3 of the wave's 32
  // rows (tiles 0, 1) and the same up rows (tiles 2, 3) for pairs i and 16 + i. h = act(gate +
  // b_g, up + b_u) x routing weight is formed in registers and the wave's 32 rows of each pair,
  // one block of the down input image, are split there: the lane holds split lanes 2g and 2g+1
  // (elements 4g, 4g+16, 4g+1, 4g+17 and 4g+2, 4g+18, 4g+3, 4g+19; the split of k_split_rows),
  // the block's other elements are in lanes xor 16 and xor 32.
  const int lr0 = wave * (kTR * 16);  // the wave's first row within the item (bias_s index)
  const int nbM = a.M >> 5;
#pragma unroll
  for (int pg = 0; pg < kPG; ++pg) {
    const int pl = pg * 16 + i;
    const float pw = bias_s[2 * kRows + min(pl, kPairTile - 1)];
    float hv[2][4];  // [tile][r]: row 16 tile + 4g + r
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int lr = lr0 + 16 * t2 + 4 * g + r;
        float gv = acc[t2][pg][r], uv = acc[2 + t2][pg][r];
        if (a.b0) gv = gv + bias_s[lr];
        if (a.b1) uv = uv + bias_s[kRows + lr];
        hv[t2][r] = (a.act == MR_ACT_SWIGLU_OAI ? swiglu_oai(gv, uv, a.alpha, a.limit) : silu_mul(gv, uv)) * pw;
      }
    uint32_t ca[kTerms], cb[kTerms], scales;
    split_block_x2<kGemmTerms>(hv[0][0], hv[1][0], hv[0][1], hv[1][1], hv[0][2], hv[1][2], hv[0][3], hv[1][3], ca, cb,
                               scales);
    if (pl < np && wrow0 < a.M) {  // M % 32 == 0: the wave's 32 rows are all inside
      const size_t bi = (size_t)(p0 + pl) * nbM + (wrow0 >> 5);
      uint32_t* dst = reinterpret_cast<uint32_t*>(a.himg + bi * kImgBytes);
#pragma unroll
      for (int t = 0; t < kGemmTerms; ++t)
        *reinterpret_cast<uint2*>(dst + t * 8 + 2 * g) = make_uint2(ca[t], cb[t]);
      if (g == 0) a.hsc[bi] = scales;
    }
  }
}

// ---- combine -----------------------------------------------------------------------------
// y[t][row] = sum over t's pairs in ascending pair index (= ascending expert) of
// o[pair][row] + w * b_down[e][row], then + sig[t] * o_sh[t][row] when a shared expert ran
// (layer.rs:1935-1951). One thread per (token, 4 rows) on a (row groups, tokens) grid (tokens
// past gridDim.y loop); the token's (at most KM) pair indices stay in registers and are taken
// smallest first, and all of a thread's loads issue before the sums. H % 4 == 0.
template <int KM>
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ o, const int32_t* __restrict__ pair_of,
                                                 const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                 const float* __restrict__ down_b, int T, int k, int H,
                                                 const float* __restrict__ o_sh, const float* __restrict__ sh_sig,
                                                 float* __restrict__ y) {
  const int row = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (row >= H) return;
  for (int t = blockIdx.y; t < T; t += gridDim.y) {
    int ps[KM];
#pragma unroll
    for (int s = 0; s < KM; ++s) ps[s] = s < k ? pair_of[t * k + s] : INT_MAX;
    f32x4 v[KM], bv[KM];
    float wv[KM];
#pragma unroll
    for (int r = 0; r < KM; ++r) {
      if (r < k) {
        int best = INT_MAX, bs = 0;
#pragma unroll
        for (int s = 0; s < KM; ++s)
          if (ps[s] < best) best = ps[s], bs = s;
#pragma unroll
        for (int s = 0; s < KM; ++s)
          if (s == bs) ps[s] = INT_MAX;
        v[r] = *reinterpret_cast<const f32x4*>(o + (size_t)best * H + row);
        if (down_b) {
          wv[r] = w[t * k + bs];
          bv[r] = *reinterpret_cast<const f32x4*>(down_b + (size_t)idx[t * k + bs] * H + row);
        }
      }
    }
    f32x4 sv = {0.f, 0.f, 0.f, 0.f};
    float sg = 0.f;
    if (o_sh) {
      sv = *reinterpret_cast<const f32x4*>(o_sh + (size_t)t * H + row);
      sg = sh_sig[t];
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < KM; ++r) {
      if (r < k) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float x = v[r][c];
          if (down_b) x = x + wv[r] * bv[r][c];
          acc[c] = acc[c] + x;
        }
      }
    }
    if (o_sh)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = acc[c] + sg * sv[c];
    *reinterpret_cast<f32x4*>(y + (size_t)t * H + row) = acc;
  }
}

// ---- host side -------------------------------------------------------------------------------
namespace {
constexpr uint64_t kAlign = 256;
uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
struct GroupedPlan {
  uint64_t pair_tok, pair_w, pair_of, exp_off, tile_off, img_x, sc_x, img_h, sc_h, obuf;
  uint64_t img_hsh, sc_hsh, osh, sig, total;
};
GroupedPlan grouped_plan(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish) {
  GroupedPlan p{};
  const uint64_t P = T * k;
  uint64_t o = 0;
  p.pair_tok = o, o += up(P * 4);
  p.pair_w = o, o += up(P * 4);
  p.pair_of = o, o += up(P * 4);
  p.exp_off = o, o += up((E + 1) * 4);
  p.tile_off = o, o += up((E + 1) * 4);
  p.img_x = o, o += up(T * (H / 32) * kImgBytes);
  p.sc_x = o, o += up(T * (H / 32) * 4);
  p.img_h = o, o += up(P * (I / 32) * kImgBytes);
  p.sc_h = o, o += up(P * (I / 32) * 4);
  p.obuf = o, o += up(P * H * 4);
  p.img_hsh = o, o += up(T * (Ish / 32) * kImgBytes);  // the shared expert (Ish = 0: none)
  p.sc_hsh = o, o += up(T * (Ish / 32) * 4);
  p.osh = o, o += up(Ish ? T * H * 4 : 0);
  p.sig = o, o += up(Ish ? T * 4 : 0);
  p.total = o;
  return p;
}
}  // namespace

uint64_t grouped_scratch_bytes(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H, uint64_t Ish) {
  return grouped_plan(T, k, E, I, H, Ish).total;
}

GroupedScratch grouped_scratch(const Scratch& s, uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H,
                               uint64_t Ish) {
  const GroupedPlan p = grouped_plan(T, k, E, I, H, Ish);
  char* b = static_cast<char*>(s.grouped);
  GroupedScratch g{};
  g.pair_tok = reinterpret_cast<int32_t*>(b + p.pair_tok);
  g.pair_w = reinterpret_cast<float*>(b + p.pair_w);
  g.pair_of = reinterpret_cast<int32_t*>(b + p.pair_of);
  g.exp_off = reinterpret_cast<int32_t*>(b + p.exp_off);
  g.tile_off = reinterpret_cast<int32_t*>(b + p.tile_off);
  g.img_x = reinterpret_cast<uint8_t*>(b + p.img_x);
  g.sc_x = reinterpret_cast<uint32_t*>(b + p.sc_x);
  g.img_h = reinterpret_cast<uint8_t*>(b + p.img_h);
  g.sc_h = reinterpret_cast<uint32_t*>(b + p.sc_h);
  g.obuf = reinterpret_cast<float*>(b + p.obuf);
  g.img_hsh = reinterpret_cast<uint8_t*>(b + p.img_hsh);
  g.sc_hsh = reinterpret_cast<uint32_t*>(b + p.sc_hsh);
  g.osh = reinterpret_cast<float*>(b + p.osh);
  g.sig = reinterpret_cast<float*>(b + p.sig);
  return g;
}
// MXFP4 routed experts, and an MXFP4 shared expert of any width (a multiple of 32), which runs
// as one more group: every token, weight 1, SiLU, then its sigmoid gate in the combine.
bool grouped_supported(const mr_layer& L) {
  if (L.type != MR_GGML_MXFP4 || L.d.top_k > 16 || L.H % 32 != 0 || L.I % 32 != 0 || L.E > 1024 ||
      L.H > 4u * 32 * kMaxSteps || L.I > 4u * 32 * kMaxSteps)
    return false;
  if (L.d.sh_gate && (L.d.sh_gate->type != MR_GGML_MXFP4 || L.d.sh_up->type != MR_GGML_MXFP4 ||
                      L.d.sh_down->type != MR_GGML_MXFP4 || L.Ish == 0 || L.Ish % 32 != 0 ||
                      L.Ish > 4u * 32 * kMaxSteps))
    return false;
  return true;
}

hipError_t launch_group(const Launch& K, const int32_t* idx, const float* w, int P, int k, int E, int32_t* pair_tok,
                        float* pair_w, int32_t* pair_of, int32_t* exp_off, int32_t* tile_off) {
  ProfScope ps(K, "group");
  hipLaunchKernelGGL(k_group, dim3(1), dim3(256), 0, K.s, idx, w, P, k, E, pair_tok, pair_w, pair_of, exp_off,
                     tile_off);
  return hipGetLastError();
}

hipError_t launch_combine(const Launch& K, const float* o, const int32_t* pair_of, const int32_t* idx, const float* w,
                          const float* down_b, uint32_t T, int k, int H, const float* o_sh, const float* sh_sig,
                          float* y) {
  ProfScope ps(K, "combine");
  const dim3 grid((unsigned)((H / 4 + 255) / 256), std::min<uint32_t>(T, 65535u));
  if (k <= 4)
    hipLaunchKernelGGL(k_combine<4>, grid, dim3(256), 0, K.s, o, pair_of, idx, w, down_b, (int)T, k, H, o_sh, sh_sig,
                       y);
  else if (k <= 8)
    hipLaunchKernelGGL(k_combine<8>, grid, dim3(256), 0, K.s, o, pair_of, idx, w, down_b, (int)T, k, H, o_sh, sh_sig,
                       y);
  else
    hipLaunchKernelGGL(k_combine<16>, grid, dim3(256), 0, K.s, o, pair_of, idx, w, down_b, (int)T, k, H, o_sh,
                       sh_sig, y);
  return hipGetLastError();
}

// Workgroups for a grouped GEMM of at most `items` work items: a multiple of the XCD count, so
// that every XCD's contiguous range of ceil(n_work / 8) items has a workgroup for each item
// (workgroup b takes item (b mod 8) * ceil(n_work / 8) + b / 8).
unsigned grouped_grid(uint64_t items) { return (unsigned)((items + kXcds - 1) / kXcds * kXcds); }

hipError_t launch_grouped(const Launch& K, const mr_layer& L, const float* x, uint32_t T, const int32_t* idx,
                          const float* w, float* y, const GroupedScratch& gs) {
  const int k = (int)L.d.top_k, E = (int)L.E, H = (int)L.H, I = (int)L.I;
  const int P = (int)T * k;
  const int max_tiles = (P + kPairTile - 1) / kPairTile + E;
  hipError_t e;
  if ((e = launch_group(K, idx, w, P, k, E, gs.pair_tok, gs.pair_w, gs.pair_of, gs.exp_off, gs.tile_off)) !=
      hipSuccess)
    return e;
  {
    ProfScope ps(K, "split_x");
    hipLaunchKernelGGL(k_split_rows, dim3((unsigned)((H / 32 + 31) / 32), std::min<uint32_t>(T, 65535u)), dim3(256), 0,
                       K.s, x, (int)T, H, gs.img_x, gs.sc_x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  GroupedArgs a{};
  a.w0 = expert_loc(L.d.gate), a.w1 = expert_loc(L.d.up);
  a.b0 = L.d.gate_bias, a.b1 = L.d.up_bias;
  a.img = gs.img_x, a.isc = gs.sc_x, a.pair_tok = gs.pair_tok, a.pair_w = gs.pair_w;
  a.exp_off = gs.exp_off, a.tile_off = gs.tile_off, a.himg = gs.img_h, a.hsc = gs.sc_h;
  a.M = I, a.K = H, a.E = E;
  a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  {
    ProfScope ps(K, "grouped_gateup");
    constexpr int rows = kRowsOf<true>;
    hipLaunchKernelGGL(k_grouped_gemm<true>, dim3(grouped_grid((uint64_t)((I + rows - 1) / rows) * max_tiles)), dim3(kGW * 64), 0,
                       K.s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  GroupedArgs d{};
  d.w0 = expert_loc(L.d.down);
  d.img = gs.img_h, d.isc = gs.sc_h, d.pair_tok = nullptr, d.pair_w = gs.pair_w;
  d.exp_off = gs.exp_off, d.tile_off = gs.tile_off, d.out = gs.obuf;
  d.M = H, d.K = I, d.E = E;
  {
    ProfScope ps(K, "grouped_down");
    constexpr int rows = kRowsOf<false>;
    hipLaunchKernelGGL(k_grouped_gemm<false>, dim3(grouped_grid((uint64_t)((H + rows - 1) / rows) * max_tiles)), dim3(kGW * 64), 0,
                       K.s, d);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (!L.d.sh_gate) return launch_combine(K, gs.obuf, gs.pair_of, idx, w, L.d.down_bias, T, k, H, nullptr, nullptr, y);
  // The shared expert (layer.rs:1898-1953): one group of every token on the same x images,
  // weight 1 and SiLU (the routed experts' activation does not apply), its down outputs
  // [T][H], then sigmoid(x . gate_inp) per token, which the combine applies after the routed
  // sum.
  const int Ish = (int)L.Ish, tiles = ((int)T + kPairTile - 1) / kPairTile;
  GroupedArgs sg{};
  sg.w0 = expert_loc(L.d.sh_gate), sg.w1 = expert_loc(L.d.sh_up);
  sg.img = gs.img_x, sg.isc = gs.sc_x, sg.single_p = (int)T;
  sg.himg = gs.img_hsh, sg.hsc = gs.sc_hsh;
  sg.M = Ish, sg.K = H, sg.E = 1, sg.act = MR_ACT_SILU;
  {
    ProfScope ps(K, "grouped_shared_gateup");
    constexpr int rows = kRowsOf<true>;
    hipLaunchKernelGGL(k_grouped_gemm<true>, dim3(grouped_grid((uint64_t)((Ish + rows - 1) / rows) * tiles)),
                       dim3(kGW * 64), 0, K.s, sg);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  GroupedArgs sd{};
  sd.w0 = expert_loc(L.d.sh_down);
  sd.img = gs.img_hsh, sd.isc = gs.sc_hsh, sd.single_p = (int)T, sd.out = gs.osh;
  sd.M = H, sd.K = Ish, sd.E = 1;
  {
    ProfScope ps(K, "grouped_shared_down");
    constexpr int rows = kRowsOf<false>;
    hipLaunchKernelGGL(k_grouped_gemm<false>, dim3(grouped_grid((uint64_t)((H + rows - 1) / rows) * tiles)),
                       dim3(kGW * 64), 0, K.s, sd);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if ((e = launch_sh_gate(K, x, T, H, L.d.sh_gate_inp, gs.sig)) != hipSuccess) return e;
  return launch_combine(K, gs.obuf, gs.pair_of, idx, w, L.d.down_bias, T, k, H, gs.osh, gs.sig, y);
}

}  // namespace mr
