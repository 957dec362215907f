// mr_grouped.hip -- multi-token (prefill / batched) MXFP4 MoE experts as grouped
// GEMMs on the gfx950 scaled MX-fp4 MFMA.
//
// The reference runs each expert once over all of its tokens: index_select of
// the expert's tokens, gate/up/act/down, x routing weight, index_add back
// (layer.rs:2148-2183; CPU: mxfp4_matmul per expert, layer.rs:1449-1514). Here:
//   k_group       (token, slot) pairs sorted by (expert, token, slot); per-expert
//                 pair offsets and 32-pair tile offsets; pair index of every
//                 (token, slot).
//   k_split_rows  activation rows -> e4m3 B images (4 terms per 32-element block).
//   k_grouped_gemm<true>   gate and up for one (expert, 64-row tile, 32-pair tile):
//                 A = native MXFP4 weight rows, B = the 16 pairs' x images; epilogue
//                 bias + activation x routing weight -> h [pair][I].
//   k_grouped_gemm<false>  down for one (expert, 128-row tile, 32-pair tile) on the
//                 h images -> o [pair][H].
//   k_combine     y[t] = sum over t's pairs in ascending expert order of
//                 (o + w*b_down) (the order of layer.rs:1092-1106).
// Every weight byte of an expert is read by the ceil(n_e/16) pair tiles of its
// row tiles; work items are laid out so those repeats, and the repeats of the
// pairs' activation images over row tiles, hit the same XCD's L2.
#include "mr_device.h"
#include "mr_fused_common.h"
#include "mr_internal.h"
#include "mr_mx_mfma.h"

#include <algorithm>

namespace mr {

constexpr int kPairTile = 32;   // pairs (tokens) per work item = 8 MFMA column groups x 4
constexpr int kXcds = 8;        // MI355X accelerator complex dies (one L2 each)
constexpr int kMaxSteps = 32;   // K steps (4 blocks) per row: K <= 4096

// ---- grouping ---------------------------------------------------------------------------
// One workgroup. Positions inside an expert follow (token, slot) order, so the
// result does not depend on thread timing.
__global__ __launch_bounds__(256) void k_group(const int32_t* __restrict__ idx, const float* __restrict__ w,
                                               int P, int k, int E, int32_t* __restrict__ pair_tok,
                                               float* __restrict__ pair_w, int32_t* __restrict__ pair_of,
                                               int32_t* __restrict__ exp_off, int32_t* __restrict__ tile_off) {
  __shared__ int cnt[1024];
  __shared__ int run[1024];
  __shared__ int ce[256];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 256) cnt[e] = 0, run[e] = 0;
  __syncthreads();
  for (int q = tid; q < P; q += 256) atomicAdd(&cnt[min(max(idx[q], 0), E - 1)], 1);
  __syncthreads();
  if (tid == 0) {
    int po = 0, to = 0;
    for (int e = 0; e < E; ++e) {
      exp_off[e] = po, tile_off[e] = to;
      po += cnt[e], to += (cnt[e] + kPairTile - 1) / kPairTile;
      cnt[e] = exp_off[e];  // reuse as the expert's base
    }
    exp_off[E] = po, tile_off[E] = to;
  }
  __syncthreads();
  for (int base = 0; base < P; base += 256) {
    const int q = base + tid;
    const int e = q < P ? min(max(idx[q], 0), E - 1) : -1;
    ce[tid] = e;
    __syncthreads();
    if (e >= 0) {
      int rank = 0;
      for (int j = 0; j < tid; ++j) rank += ce[j] == e ? 1 : 0;
      const int pos = cnt[e] + run[e] + rank;
      pair_tok[pos] = q / k, pair_w[pos] = w[q], pair_of[q] = pos;
    }
    __syncthreads();
    if (e >= 0) atomicAdd(&run[e], 1);
    __syncthreads();
  }
}

// ---- activation rows -> B images ------------------------------------------------------------
// Row r of `src` (D floats) -> img[r][D/32][kImgBytes] + sc[r][D/32]; 8 lanes per block.
__global__ __launch_bounds__(256) void k_split_rows(const float* __restrict__ src, int n_rows, int D,
                                                    uint8_t* __restrict__ img, uint32_t* __restrict__ sc) {
  const int nb = D >> 5;
  const long long blk = (long long)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int m = threadIdx.x & 7;
  const bool in = blk < (long long)n_rows * nb;
  const long long bb = in ? blk : 0;
  const float* p = src + (bb / nb) * (long long)D + (bb % nb) * 32 + 2 * m;
  const f32x2 lo = *reinterpret_cast<const f32x2*>(p);       // elements 2m, 2m+1
  const f32x2 hi = *reinterpret_cast<const f32x2*>(p + 16);  // elements 2m+16, 2m+17
  uint32_t codes[kTerms], scales;
  split_block8(lo.x, hi.x, lo.y, hi.y, codes, scales);
  if (in) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(img + bb * kImgBytes);
#pragma unroll
    for (int t = 0; t < kTerms; ++t) dst[t * 8 + m] = codes[t];
    if (m == 0) sc[bb] = scales;
  }
}

// ---- grouped GEMM -------------------------------------------------------------------------
struct GroupedArgs {
  const uint8_t* w0;  // gate (GATEUP) or down
  const uint8_t* w1;  // up (GATEUP)
  const uint64_t* off0;
  const uint64_t* off1;
  const float* b0;  // gate bias [E][M] (GATEUP) or null
  const float* b1;  // up bias
  const uint8_t* img;    // B images [rows][K/32][kImgBytes]
  const uint32_t* isc;   // [rows][K/32]
  const int32_t* pair_tok;  // B row of pair p (GATEUP: its token) or null (row = p)
  const float* pair_w;
  const int32_t* exp_off;
  const int32_t* tile_off;
  float* out;  // [P][M]
  int M, K, E, max_tiles;
  int act;
  float alpha, limit;
};

// Grouped GEMM work item: (expert e, row tile, 32-pair tile). 8 waves; each wave owns
// 16 output rows of one matrix (gate/up: waves 0-3 gate, 4-7 up, the same 64 rows;
// down: 8 x 16 = 128 rows) and all 32 pairs (8 MFMA column groups of 4 pairs x 4 terms).
// K advances one MFMA step (4 blocks) at a time through double-buffered LDS:
//   B: the step's 32 pairs x 4 blocks x 128-byte images (16 KB), loaded cooperatively
//      by direct global->LDS loads (each pair's 512 bytes are contiguous) and shared
//      by the 8 waves;
//   A: each wave's 16 rows x 68 bytes, fetched as 6 aligned 16-byte pieces per row by
//      direct global->LDS loads (rows are 1530 bytes apart, so a wave load covers ~10
//      rows' contiguous bytes instead of 16 scattered block windows).
constexpr int kGemmWaves = 8;
constexpr int kAPieces = 6;                         // pieces per row and step: 15 + 68 + 3 <= 96
constexpr int kAStage = 2 * 1024;                   // one A buffer: 96 pieces + pad (2 wave loads)
constexpr int kBStage = kPairTile * 4 * kImgBytes;  // one B buffer: 32 pairs x 4 blocks
static_assert(kPairTile * 4 * 8 == 2 * 512, "two B pieces per thread per step");

template <bool GATEUP>
__global__ __launch_bounds__(512, 2) void k_grouped_gemm(GroupedArgs a) {
  __shared__ __align__(16) uint8_t bst[2][kBStage];
  __shared__ __align__(16) uint32_t bsc[2][kPairTile * 4];
  __shared__ __align__(16) uint8_t ast[kGemmWaves][2][kAStage];
  __shared__ __align__(16) uint8_t zero[32];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int i = lane & 15, g = lane >> 4, t = i & 3;
  constexpr int NM = GATEUP ? 2 : 1;
  constexpr int kRows = 16 * kGemmWaves / NM;  // rows per work item
  // Work items are ordered (expert, row tile, pair tile of the expert), and each
  // XCD (workgroups are dispatched round-robin over kXcds) takes one contiguous
  // range of them: the items that share an expert's row tile (A) or its pairs'
  // images (B) run on the same XCD and meet in its L2.
  const int n_rt = (a.M + kRows - 1) / kRows;
  const int n_work = n_rt * a.tile_off[a.E];
  const int per_xcd = (n_work + kXcds - 1) / kXcds;
  const int loc = blockIdx.x / kXcds;
  const int w = (blockIdx.x % kXcds) * per_xcd + loc;
  if (loc >= per_xcd || w >= n_work) return;  // uniform: no work item for this workgroup
  int lo = 0, hi = a.E;  // expert: n_rt * tile_off[e] <= w < n_rt * tile_off[e+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (n_rt * a.tile_off[mid] <= w) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int nt_e = a.tile_off[e + 1] - a.tile_off[e];
  const int wl = w - n_rt * a.tile_off[e];
  const int rt = wl / nt_e, tl = wl - rt * nt_e;
  const int p0 = a.exp_off[e] + tl * kPairTile;
  const int np = min(kPairTile, a.exp_off[e + 1] - p0);
  if (tid < 8) reinterpret_cast<uint32_t*>(zero)[tid] = 0u;

  const int nbK = a.K >> 5, S = (nbK + 3) >> 2;
  const uint64_t rb = (uint64_t)nbK * 17;
  const int m = GATEUP ? (wave >> 2) : 0;
  const int row0 = rt * kRows + (GATEUP ? (wave & 3) : wave) * 16;
  const bool rows_in = row0 < a.M;          // wave-uniform; other waves still load B and sync
  const int row0c = min(row0, a.M - 16);    // M is a multiple of 16
  const uint8_t* W = (m ? a.w1 + a.off1[e] : a.w0 + a.off0[e]) + (uint64_t)row0c * rb;
  // this thread's B pieces (q = j*512 + tid): pair q/32, block (q/8)%4, part q%8
  const uint8_t* bsrc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = j * 512 + tid;
    const int p = p0 + min(q >> 5, np - 1);
    const int r = a.pair_tok ? a.pair_tok[p] : p;
    bsrc[j] = a.img + (size_t)r * nbK * kImgBytes + (q & 7) * 16;
  }
  const int sq = tid & 127;  // scale word sq (waves 0-1): pair sq/4, block sq%4
  const uint32_t* ssrc;
  {
    const int p = p0 + min(sq >> 2, np - 1);
    const int r = a.pair_tok ? a.pair_tok[p] : p;
    ssrc = a.isc + (size_t)r * nbK;
  }
  // A pieces of this wave (p = it*64 + lane): row p/6, piece p%6 (p >= 96: pad)
  const uint8_t* arow[2];
  int apc[2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int pp = it * 64 + lane;
    const int r = min(pp / kAPieces, 15);
    apc[it] = min(pp - r * kAPieces, kAPieces - 1);
    arow[it] = W + (uint64_t)r * rb;
  }
  const uintptr_t my_row = reinterpret_cast<uintptr_t>(W + (uint64_t)i * rb);

  auto issue = [&](int st, int buf) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const uintptr_t first = reinterpret_cast<uintptr_t>(arow[it] + (size_t)(4 * st) * 17) & ~(uintptr_t)15;
      const uintptr_t last = (reinterpret_cast<uintptr_t>(arow[it] + (size_t)nbK * 17) - 1) & ~(uintptr_t)15;
      const uintptr_t src = min(first + 16 * (uintptr_t)apc[it], last);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), &ast[wave][buf][it * 1024], 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = j * 512 + tid;
      const int blk = min(4 * st + ((q >> 3) & 3), nbK - 1);
      __builtin_amdgcn_global_load_lds(bsrc[j] + (size_t)blk * kImgBytes, &bst[buf][(j * 512 + wave * 64) * 16], 16,
                                       0, 0);
    }
    if (wave < 2)
      __builtin_amdgcn_global_load_lds(ssrc + min(4 * st + (sq & 3), nbK - 1), &bsc[buf][wave * 64], 4, 0, 0);
  };

  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  issue(0, 0);
  for (int st = 0; st < S; ++st) {
    const int buf = st & 1;
    if (st + 1 < S) {
      __syncthreads();  // every wave is done with buffer buf^1 (step st-1)
      issue(st + 1, buf ^ 1);
      if (wave < 2)
        asm volatile("s_waitcnt vmcnt(5)" ::: "memory");  // step st's loads have landed
      else
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      vm_drain();
    }
    __syncthreads();  // step st's A and B are in LDS for every wave
    if (rows_in) {
      const int b = 4 * st + g;  // this lane's A block
      const int lead = (int)((my_row + (uintptr_t)(4 * st) * 17) & 15u);
      const int off = i * (kAPieces * 16) + lead + g * 17;
      const uint32_t* wp = reinterpret_cast<const uint32_t*>(&ast[wave][buf][off & ~3]);
      RawBlk ra;
      ra.d[0] = wp[0], ra.d[1] = wp[1], ra.d[2] = wp[2], ra.d[3] = wp[3], ra.d[4] = wp[4];
      const int b0 = 4 * st + (g >> 1), b1 = b0 + 2;
      const int sb_off = (b < nbK ? g : 0);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int pr = 4 * c + (i >> 2);
        const uint8_t* pb = &bst[buf][pr * 4 * kImgBytes + t * 32 + 16 * (g & 1)];
        const i32x4 v0 = *reinterpret_cast<const i32x4*>(b0 < nbK ? pb + (g >> 1) * kImgBytes : zero);
        const i32x4 v1 = *reinterpret_cast<const i32x4*>(b1 < nbK ? pb + (2 + (g >> 1)) * kImgBytes : zero);
        const i32x8 B = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        const int sb = (int)((bsc[buf][pr * 4 + sb_off] >> (8 * t)) & 0xFFu);
        acc[c] = mfma_raw(ra, (uint32_t)off & 3u, b < nbK, B, sb, acc[c]);
      }
    }
  }
  // epilogue: columns 4*tl .. 4*tl+3 of group c are the 4 terms of pair 4c+tl
  float* xch = reinterpret_cast<float*>(&bst[0][0]);  // gate results for the up waves (32 KB)
  if (GATEUP) {
    __syncthreads();  // the K loop's LDS is no longer read
    if (m == 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) xch[(((wave & 3) * 8 + c) * 4 + r) * 64 + lane] = sum4(acc[c][r]);
    }
    __syncthreads();
    if (m == 0) return;
  }
  if (!rows_in) return;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = sum4(acc[c][r]);
      const int pl = 4 * c + (i >> 2);
      const int orow = row0 + 4 * g + r;
      if (t == 0 && pl < np && orow < a.M) {
        const int p = p0 + pl;
        float o;
        if (GATEUP) {
          float gv = xch[(((wave & 3) * 8 + c) * 4 + r) * 64 + lane], uv = v;
          if (a.b0) gv = gv + a.b0[(size_t)e * a.M + orow];
          if (a.b1) uv = uv + a.b1[(size_t)e * a.M + orow];
          const float h = a.act == MR_ACT_SWIGLU_OAI ? swiglu_oai(gv, uv, a.alpha, a.limit) : silu_mul(gv, uv);
          o = h * a.pair_w[p];
        } else {
          o = v;
        }
        a.out[(size_t)p * a.M + orow] = o;
      }
    }
  }
}

// ---- combine -----------------------------------------------------------------------------
// y[t][row] = sum over t's pairs in ascending pair index (= ascending expert) of
// o[pair][row] + w * b_down[e][row]. One thread per (token, row).
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ o, const int32_t* __restrict__ pair_of,
                                                 const int32_t* __restrict__ idx, const float* __restrict__ w,
                                                 const float* __restrict__ down_b, int T, int k, int H,
                                                 float* __restrict__ y) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)T * H) return;
  const int t = (int)(gid / H), row = (int)(gid % H);
  int ps[16], ss[16];
  for (int s = 0; s < k; ++s) {  // insertion sort of the token's pairs
    const int p = pair_of[t * k + s];
    int j = s;
    while (j > 0 && ps[j - 1] > p) ps[j] = ps[j - 1], ss[j] = ss[j - 1], --j;
    ps[j] = p, ss[j] = s;
  }
  float acc = 0.f;
  for (int j = 0; j < k; ++j) {
    float v = o[(size_t)ps[j] * H + row];
    if (down_b) v = v + w[t * k + ss[j]] * down_b[(size_t)idx[t * k + ss[j]] * H + row];
    acc = acc + v;
  }
  y[gid] = acc;
}

// ---- host side -------------------------------------------------------------------------------
namespace {
constexpr uint64_t kAlign = 256;
uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
struct GroupedPlan {
  uint64_t pair_tok, pair_w, pair_of, exp_off, tile_off, img_x, sc_x, img_h, sc_h, hbuf, obuf, total;
};
GroupedPlan grouped_plan(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H) {
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
  p.hbuf = o, o += up(P * I * 4);
  p.obuf = o, o += up(P * H * 4);
  p.total = o;
  return p;
}
}  // namespace

uint64_t grouped_scratch_bytes(uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H) {
  return grouped_plan(T, k, E, I, H).total;
}

GroupedScratch grouped_scratch(const Scratch& s, uint64_t T, uint64_t k, uint64_t E, uint64_t I, uint64_t H) {
  const GroupedPlan p = grouped_plan(T, k, E, I, H);
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
  g.hbuf = reinterpret_cast<float*>(b + p.hbuf);
  g.obuf = reinterpret_cast<float*>(b + p.obuf);
  return g;
}
bool grouped_supported(const mr_layer& L) {
  return L.type == MR_GGML_MXFP4 && !L.d.sh_gate && L.d.top_k <= 16 && L.H % 32 == 0 && L.I % 32 == 0 &&
         L.E <= 1024 && L.H <= 4u * 32 * kMaxSteps && L.I <= 4u * 32 * kMaxSteps;
}

hipError_t launch_grouped(const Launch& K, const mr_layer& L, const float* x, uint32_t T, const int32_t* idx,
                          const float* w, float* y, const GroupedScratch& gs) {
  const int k = (int)L.d.top_k, E = (int)L.E, H = (int)L.H, I = (int)L.I;
  const int P = (int)T * k;
  const int max_tiles = (P + kPairTile - 1) / kPairTile + E;
  hipError_t e;
  {
    ProfScope ps(K, "group");
    hipLaunchKernelGGL(k_group, dim3(1), dim3(256), 0, K.s, idx, w, P, k, E, gs.pair_tok, gs.pair_w, gs.pair_of,
                       gs.exp_off, gs.tile_off);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    ProfScope ps(K, "split_x");
    const long long nblk = (long long)T * (H / 32);
    hipLaunchKernelGGL(k_split_rows, dim3((unsigned)((nblk + 31) / 32)), dim3(256), 0, K.s, x, (int)T, H, gs.img_x,
                       gs.sc_x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  GroupedArgs a{};
  a.w0 = L.d.gate->base, a.w1 = L.d.up->base, a.off0 = L.d.gate->d_offsets, a.off1 = L.d.up->d_offsets;
  a.b0 = L.d.gate_bias, a.b1 = L.d.up_bias;
  a.img = gs.img_x, a.isc = gs.sc_x, a.pair_tok = gs.pair_tok, a.pair_w = gs.pair_w;
  a.exp_off = gs.exp_off, a.tile_off = gs.tile_off, a.out = gs.hbuf;
  a.M = I, a.K = H, a.E = E, a.max_tiles = max_tiles;
  a.act = (int)L.d.act, a.alpha = L.d.alpha, a.limit = L.d.limit;
  {
    ProfScope ps(K, "grouped_gateup");
    hipLaunchKernelGGL(k_grouped_gemm<true>, dim3((unsigned)(((I + 63) / 64) * max_tiles)), dim3(512), 0, K.s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    ProfScope ps(K, "split_h");
    const long long nblk = (long long)P * (I / 32);
    hipLaunchKernelGGL(k_split_rows, dim3((unsigned)((nblk + 31) / 32)), dim3(256), 0, K.s, gs.hbuf, P, I, gs.img_h,
                       gs.sc_h);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  GroupedArgs d{};
  d.w0 = L.d.down->base, d.off0 = L.d.down->d_offsets;
  d.img = gs.img_h, d.isc = gs.sc_h, d.pair_tok = nullptr, d.pair_w = gs.pair_w;
  d.exp_off = gs.exp_off, d.tile_off = gs.tile_off, d.out = gs.obuf;
  d.M = H, d.K = I, d.E = E, d.max_tiles = max_tiles;
  {
    ProfScope ps(K, "grouped_down");
    hipLaunchKernelGGL(k_grouped_gemm<false>, dim3((unsigned)(((H + 127) / 128) * max_tiles)), dim3(512), 0, K.s, d);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    ProfScope ps(K, "combine");
    const long long n = (long long)T * H;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, K.s, gs.obuf, gs.pair_of, idx, w,
                       L.d.down_bias, (int)T, k, H, y);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mr
