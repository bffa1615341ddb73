// Batched FP16 leaf products on CDNA4 MFMA (gfx950).
//
//   P[r] = A'[r] @ B'[r]^T,   A'[r]: [Mb, Kb], B'[r]: [Nb, Kb] in the operand layout of
//   fastmm_device.h (K-slab-major when Kb % 32 == 0, else row-major); P row-major.
//
// Fast kernel (Kb % 32 == 0, Kb >= 96, 16-byte aligned operands): one
// workgroup = 4 waves (one per SIMD) owns a 256 x 256 tile of one leaf; each
// wave owns 128 x 128 as 4 x 4 v_mfma_f32_32x32x16_f16 accumulators (all 256
// AGPRs). K advances in 32-wide slices through a 4-slot LDS ring filled by
// direct-to-LDS loads (global_load_lds_dwordx4) three slices ahead, so a slice's
// global latency is covered by three slices of MFMAs and no VGPRs stage data.
// Per slice: the fragments of its second k-step are read while the first
// k-step's MFMAs run; after a partial vmcnt wait (the next slice is resident)
// and one barrier, the refill of the ring slot freed one slice earlier is
// issued and the next slice's first fragments are read under the second
// k-step's MFMAs. The refill is safe after that barrier because every wave
// consumed (and waited for) its reads of the freed slot during the previous
// slice.
//
// LDS layout: a slice row is 32 halves = 64 bytes = 4 chunks of 16 bytes;
// chunk c of row r sits at c ^ ((r >> 2) & 3). gfx950's LDS is 64 banks wide,
// so the 16 lanes of one ds_read_b128 phase (16 consecutive rows, one k) hit 16
// distinct (row % 4, chunk) bank groups; the DMA writes 1 KB contiguous per
// instruction (lane L -> slot L), so the swizzle is applied by choosing which
// global chunk each lane fetches. In the K-slab layout those 16 rows of one
// slab are also 1 KB of consecutive global bytes.
//
// MFMA operands are passed as (B', A'): lane l supplies B'[n l%32][k 8*(l/32)
// .. +7] and A'[m l%32][same k], so the accumulator holds P^T in the 32x32
// layout and lane l, element e is P[m l%32][n 8*(e/4) + 4*(l/32) + e%4]: four
// consecutive columns per lane. fp32 products leave as 16-byte stores; fp16
// products are staged through LDS (row pitch 264 halves: 32 rows of 8-byte
// writes spread over all 64 banks) and leave as coalesced 16-byte row
// segments.
//
// When Kb % 128 == 0 a 16x16x32 variant of the fast kernel (below, with its
// own notes) runs instead; the 32x32x16 kernel covers the other fast shapes.
// On that path, 16-bit products over more than one round of tiles run on its
// persistent form (one workgroup per CU streaming slices across tile
// boundaries, see persistent_kernel), and a last partial round of tiles can
// be split along K into fp32 parts in caller-owned scratch and added by
// tail_reduce_kernel (the split-K tail, see tail_split and launch_mfma16). A
// last tile row of at most 16 rows runs fused into the persistent kernel (its
// strip form) or in thin_rows_kernel (see leaf_plan); products beyond 1 GiB
// are stored with the non-temporal hint.
//
// Generic kernel (any Kb, any alignment): 256 x 256 tile, BK = 64, register-
// staged loads with zero fill, double-buffered LDS; used for small or ragged
// shapes where the fast kernel's preconditions fail.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "abi_common.h"
#include "fastmm_device.h"

namespace fastmm {

constexpr int kGemmThreads = 256;
constexpr int kTile = 256;

// Logical tile -> (leaf, tile row, tile column): walk the tiles of a leaf in
// groups of `group` tile rows, column by column.
__device__ __forceinline__ void tile_of(int logical, int tiles_m, int tiles_n, int group, int& leaf, int& tm,
                                        int& tn) {
  const int per_leaf = tiles_m * tiles_n;
  leaf = logical / per_leaf;
  const int t = logical - leaf * per_leaf;
  const int g = t / (group * tiles_n);
  const int first_m = g * group;
  const int rows_in_group = min(group, tiles_m - first_m);
  const int within = t - g * group * tiles_n;
  tm = first_m + within % rows_in_group;
  tn = within / rows_in_group;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w runs on
// XCD w % 8); each XCD works on a contiguous range of the logical tiles
// (tiles of one leaf share A'/B' rows in that XCD's L2): with q = total / 8
// and r = total % 8, XCD x takes q + 1 tiles if x < r, else q, starting at
// x*(q+1) (x < r) or r*(q+1) + (x-r)*q.
constexpr int kXcds = 8;

__device__ __forceinline__ void xcd_range(int total, int x, int& start, int& count) {
  const int q = total / kXcds, r = total - q * kXcds;
  start = x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  count = x < r ? q + 1 : q;
}

// One workgroup per tile: workgroup w takes tile w / 8 of its XCD's range.
__device__ __forceinline__ void decode_tile(int wg, int total, int tiles_m, int tiles_n,
                                            int group, int& leaf, int& tm, int& tn) {
  int start, count;
  xcd_range(total, wg % kXcds, start, count);
  tile_of(start + wg / kXcds, tiles_m, tiles_n, group, leaf, tm, tn);
}

// 32x32x16 MFMA on 8 operand elements per lane, fp16 or bf16 (same register
// bits, different instruction).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int kIn>
__device__ __forceinline__ float16v mfma_32x32x16(half8 a, half8 b, float16v c) {
  if constexpr (kIn == kBF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
}

// ----------------------------------------------------------------- fast path

namespace fast {

constexpr int BK = 32;
constexpr int STAGES = 4;
constexpr int STAGE_HALVES = 2 * kTile * BK;
constexpr int SEGMENTS = kTile / 16 / 4;  // 1 KB segments per operand per wave
constexpr int OUT_PITCH = kTile + 8;       // halves per staged output row
constexpr int LDS_BYTES = (STAGES * STAGE_HALVES * 2 > kTile * OUT_PITCH * 2)
                              ? STAGES * STAGE_HALVES * 2
                              : kTile * OUT_PITCH * 2;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else static_assert(N < 0, "unsupported vmcnt");
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef const void __attribute__((address_space(1)))* global_ptr;
typedef void __attribute__((address_space(3)))* lds_ptr;

template <int kIn, int kOut>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void leaf_gemm_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                      void* __restrict__ P, int Mb, int Nb, int Kb, int tiles_m, int tiles_n,
                      int total_tiles) {
  constexpr int TM = 4, TN = 4;  // 32x32 accumulators per wave (128 x 128)
  extern __shared__ __attribute__((aligned(16))) half_t smem[];

  int leaf, tm, tn;
  decode_tile(blockIdx.x, total_tiles, tiles_m, tiles_n, 8, leaf, tm, tn);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = tm * kTile, n0 = tn * kTile;
  const half_t* a_leaf = A + static_cast<int64_t>(leaf) * Mb * Kb;
  const half_t* b_leaf = B + static_cast<int64_t>(leaf) * Nb * Kb;

  // DMA mapping: lane L of segment q writes row 16*q' + L/4, physical chunk L%4
  // (q' = 4q + wave); it fetches the logical chunk stored there. Operands are
  // K-slab-major (Kb % 32 == 0), so a segment is 1 KB of consecutive bytes.
  // Rows past the leaf are clamped onto its last row: they only feed outputs
  // that are masked.
  const int seg_row = lane >> 2;
  int a_off[SEGMENTS], b_off[SEGMENTS];
#pragma unroll
  for (int q = 0; q < SEGMENTS; ++q) {
    const int row = (q * 4 + wave) * 16 + seg_row;
    const int chunk = (lane & 3) ^ ((row >> 2) & 3);
    a_off[q] = min(m0 + row, Mb - 1) * kSlab + chunk * 8;
    b_off[q] = min(n0 + row, Nb - 1) * kSlab + chunk * 8;
  }
  const int lane_row = lane & 31, lane_half = lane >> 5;
  int rd_off[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    rd_off[ks] = lane_row * BK + (((2 * ks + lane_half) ^ ((lane_row >> 2) & 3)) << 3);
  }
  const int a_rd = wm * 128 * BK, b_rd = wn * 128 * BK;

  half8 fa[2][TM], fb[2][TN];
  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto load_slice = [&](int kt) {
    half_t* as = smem + (kt % STAGES) * STAGE_HALVES;
    half_t* bs = as + kTile * BK;
    const half_t* a_slab = a_leaf + static_cast<int64_t>(kt) * Mb * kSlab;
    const half_t* b_slab = b_leaf + static_cast<int64_t>(kt) * Nb * kSlab;
#pragma unroll
    for (int q = 0; q < SEGMENTS; ++q) {
      __builtin_amdgcn_global_load_lds((global_ptr)(a_slab + a_off[q]),
                                       (lds_ptr)(as + (q * 4 + wave) * 16 * BK), 16, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < SEGMENTS; ++q) {
      __builtin_amdgcn_global_load_lds((global_ptr)(b_slab + b_off[q]),
                                       (lds_ptr)(bs + (q * 4 + wave) * 16 * BK), 16, 0, 0);
    }
  };
  auto read_fragments = [&](int kt, int ks, int slot) {
    const half_t* as = smem + (kt % STAGES) * STAGE_HALVES;
    const half_t* bs = as + kTile * BK;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      fa[slot][i] = *reinterpret_cast<const half8*>(as + a_rd + i * 32 * BK + rd_off[ks]);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      fb[slot][j] = *reinterpret_cast<const half8*>(bs + b_rd + j * 32 * BK + rd_off[ks]);
    }
  };
  auto mfma = [&](int slot) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = mfma_32x32x16<kIn>(fb[slot][j], fa[slot][i], acc[i][j]);
  };
  // The 8 fragment reads go under the first 8 MFMAs (they are needed one
  // k-step later); the refill loads, when present, under the second half.
  auto schedule = [&](bool with_loads) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if (with_loads) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
    } else {
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }
  };

  const int nk = Kb / BK;  // >= 3, checked by the launcher
  load_slice(0);
  load_slice(1);
  load_slice(2);
  wait_vmcnt<16>();
  barrier();
  read_fragments(0, 0, 0);

  // kRefill: slice kt+3 exists; kNext: slice kt+1 exists; kWait: loads that may
  // stay in flight while slice kt+1 must be resident (those of slice kt+2).
  auto step = [&](int kt, auto refill_tag, auto next_tag, auto wait_tag) {
    constexpr bool kRefill = decltype(refill_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value;
    constexpr int kWait = decltype(wait_tag)::value;
    read_fragments(kt, 1, 1);
    mfma(0);
    schedule(false);
    if constexpr (kNext) wait_vmcnt<kWait>();
    barrier();
    if constexpr (kRefill) load_slice(kt + 3);
    if constexpr (kNext) read_fragments(kt + 1, 0, 0);
    mfma(1);
    schedule(kRefill);
  };
  int kt = 0;
  for (; kt < nk - 3; ++kt) {
    step(kt, std::true_type{}, std::true_type{}, std::integral_constant<int, 8>{});
  }
  step(kt++, std::false_type{}, std::true_type{}, std::integral_constant<int, 8>{});
  step(kt++, std::false_type{}, std::true_type{}, std::integral_constant<int, 0>{});
  step(kt, std::false_type{}, std::false_type{}, std::integral_constant<int, 0>{});

  const int64_t leaf_offset = static_cast<int64_t>(leaf) * Mb * Nb;
  if constexpr (kOut == kFP32) {
    // lane: row m0 + wm*128 + i*32 + lane_row, 4 columns per e-group.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * 128 + i * 32 + lane_row;
      if (row >= Mb) continue;
      float* out_row = static_cast<float*>(P) + leaf_offset + static_cast<int64_t>(row) * Nb;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = n0 + wn * 128 + j * 32 + 8 * g + 4 * lane_half;
          if (col < Nb) {
            *reinterpret_cast<float4*>(out_row + col) =
                make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                            acc[i][j][4 * g + 3]);
          }
        }
    }
  } else {
    // Stage the 256 x 256 16-bit tile in LDS, then store 16-byte row segments.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    uint16_t* staged = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm * 128 + i * 32 + lane_row;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = wn * 128 + j * 32 + 8 * g + 4 * lane_half;
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = from_f32<kOut>(acc[i][j][4 * g + e]);
          store16<4>(staged + row * OUT_PITCH + col, h);
        }
    }
    __syncthreads();
    const int chunk = tid & 31;  // 32 chunks of 8 halves per row
    uint16_t* out = static_cast<uint16_t*>(P) + leaf_offset;
#pragma unroll 4
    for (int pass = 0; pass < kTile / 8; ++pass) {
      const int row = pass * 8 + (tid >> 5);
      const int grow = m0 + row, gcol = n0 + chunk * 8;
      if (grow < Mb && gcol < Nb) {
        uint16_t h[8];
        load16<8>(staged + row * OUT_PITCH + chunk * 8, h);
        store16<8>(out + static_cast<int64_t>(grow) * Nb + gcol, h);
      }
    }
  }
}

}  // namespace fast

// ------------------------------------------------------- 16x16x32 fast path

// Main kernel for Kb % 128 == 0. Same 256 x 256 workgroup tile, 4 waves of
// 128 x 128, 4-slot LDS ring of 32-wide K slices and 64-bank swizzle as the
// kernel above, but on v_mfma_f32_16x16x32_f16: each wave holds 8 x 8
// accumulators of 4 floats (256 AGPRs), one MFMA step consumes a whole slice,
// and per slice and wave 64 MFMAs carry 16 fragment reads (one per 4 MFMAs,
// for the next slice) and 8 ring refills (one per 8 MFMAs, four slices ahead).
// On MI355X the MFMA rate of this GEMM is limited by board power, not by issue
// slots: with random FP16 operands 16x16x32 sustains ~15 % more flop/s than
// 32x32x16 at the same power, and spreading the refills over the whole slice
// keeps the texture path from stalling the in-order MFMA issue.
//
// A slot is refilled as soon as its fragments are in registers: at the barrier
// that opens slice kt every wave has waited for its reads of slice kt's slot
// (issued during slice kt - 1), so that slot takes slice kt + 4 while slices
// kt + 2 and kt + 3 are still in flight and slice kt + 1 is resident.
//
// The main loop is written as inline asm (MFMAs, fragment reads, waits) in
// program order; the compiler's scheduler otherwise regroups the loads and
// reads around the barrier. The asm operands tie every fragment to one of two
// register sets, so no read overwrites a register an in-flight MFMA still
// sources; s_nops before the epilogue cover the MFMA-to-AGPR-read latency the
// compiler cannot see through the asm. Loads are buffer loads to LDS from the
// K-slab-major planes: a tile's slice is 16 KB of consecutive bytes.
//
// Fragment layout (16x16x32, operands passed as (B', A')): lane l supplies
// B'[n l%16][k 8*(l/16) .. +7] and A'[m l%16][same k]; accumulator element e
// of lane l is P[m l%16][n 4*(l/16) + e].

namespace mfma16 {

constexpr int BK = 32;
constexpr int STAGES = 4;
constexpr int STAGE_HALVES = 2 * kTile * BK;
constexpr int SEGMENTS = kTile / 16 / 4;
constexpr int FM = 8, FN = 8;  // 16x16 accumulators per wave (128 x 128)
constexpr int LDS_BYTES = fast::LDS_BYTES;
static_assert(STAGES * STAGE_HALVES * 2 <= LDS_BYTES, "ring must fit the LDS reservation");

typedef float float4v __attribute__((ext_vector_type(4)));
using fast::lds_ptr;
using fast::wait_vmcnt;

template <int V>
using Int = std::integral_constant<int, V>;
template <bool V>
using Bool = std::integral_constant<bool, V>;

// kPartial (the split-K tail of a launch): workgroup w computes K part
// w / tail_count (of `split` contiguous runs of whole 4-slice groups) of
// logical tile tail_base + w % tail_count, and stores the unmasked 256 x 256
// fp32 partial sum at partial + (tile * split + part) * 256 * 256 (row-major);
// tail_reduce_kernel adds the parts. Otherwise workgroup w computes the whole
// K range of one of the first total_tiles logical tiles (XCD order).
template <int kIn, int kOut, bool kPartial>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void leaf_gemm_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                      void* __restrict__ P, int Mb, int Nb, int Kb, int tiles_m, int tiles_n,
                      int total_tiles, int tail_base, int tail_count, int split) {
  extern __shared__ __attribute__((aligned(16))) half_t smem[];
  int leaf, tm, tn;
  int k_first = 0, nk = Kb / BK;  // slices; nk is a multiple of 4, checked by the launcher
  int tile_slot = 0;
  if constexpr (kPartial) {
    const int t = blockIdx.x % tail_count, part = blockIdx.x / tail_count;
    tile_of(tail_base + t, tiles_m, tiles_n, 8, leaf, tm, tn);
    const int groups = nk / 4;
    const int g0 = part * groups / split, g1 = (part + 1) * groups / split;
    k_first = 4 * g0;
    nk = 4 * (g1 - g0);
    tile_slot = t * split + part;
  } else {
    decode_tile(blockIdx.x, total_tiles, tiles_m, tiles_n, 8, leaf, tm, tn);
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = tm * kTile, n0 = tn * kTile;
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<half_t*>(A + static_cast<int64_t>(leaf) * Mb * Kb), 0, Mb * Kb * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<half_t*>(B + static_cast<int64_t>(leaf) * Nb * Kb), 0, Nb * Kb * 2, 0x00020000);

  // DMA mapping as in the 32x32 kernel: lane L of segment q writes row
  // 16*(4q + wave) + L/4, physical chunk L%4, and fetches the logical chunk
  // stored there (byte offsets within a K slab; the slab is the scalar
  // offset). Rows past the leaf get the offset 2^31, which is out of range
  // (num_records < 2^31, checked by the launcher) with or without the scalar
  // offset added, so those lanes read nothing and their LDS slots are
  // zero-filled: the padding rows then feed zeros to MFMAs whose results are
  // never stored, which costs less energy than repeating real data.
  // A lane's rows in the four segments are r0 + 64q with r0 = 16*wave + L/4,
  // and its swizzled chunk (L%4) ^ ((row/4)%4) is the same in all of them. A
  // byte offset (row*32 + chunk*8)*2 is below 64*Mb exactly when row < Mb, so
  // one per-lane base and a uniform limit give all eight offsets.
  constexpr unsigned kOutOfRange = 0x80000000u;
  constexpr unsigned kSegmentBytes = 64 * kSlab * 2;
  const unsigned lane_base =
      static_cast<unsigned>(((wave * 16 + (lane >> 2)) * kSlab + ((lane & 3) ^ ((lane >> 4) & 3)) * 8) * 2);
  const unsigned a_first = lane_base + static_cast<unsigned>(m0 * kSlab * 2);
  const unsigned b_first = lane_base + static_cast<unsigned>(n0 * kSlab * 2);
  const unsigned a_limit = static_cast<unsigned>(Mb * kSlab * 2), b_limit = static_cast<unsigned>(Nb * kSlab * 2);
  unsigned a_off[SEGMENTS], b_off[SEGMENTS];
#pragma unroll
  for (int q = 0; q < SEGMENTS; ++q) {
    const unsigned a = a_first + q * kSegmentBytes, b = b_first + q * kSegmentBytes;
    a_off[q] = a < a_limit ? a : kOutOfRange;
    b_off[q] = b < b_limit ? b : kOutOfRange;
  }
  // Fragment reads: row l%16 of a 16-row block, logical chunk l/16. Two base
  // addresses (slots {0,1} and {2,3}) keep every offset an immediate.
  const int fr = lane & 15, fc = lane >> 4;
  const int rd = fr * BK + ((fc ^ ((fr >> 2) & 3)) << 3);
  unsigned base_a[2], base_b[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // address-space casts: generic -> LDS pointer -> 32-bit LDS byte address
    base_a[h] = (unsigned)(uintptr_t)(lds_ptr)(smem + h * 2 * STAGE_HALVES + wm * 128 * BK + rd);
    base_b[h] = (unsigned)(uintptr_t)(lds_ptr)(smem + h * 2 * STAGE_HALVES + kTile * BK + wn * 128 * BK + rd);
  }

  half8 fa[2][FM], fb[2][FN];
  float4v acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      fa[s][i] = half8{};
      fb[s][i] = half8{};
    }

  // idx 0..3: A' segments, 4..7: B' segments of slice kt into ring slot `slot`
  auto load_one = [&](int kt, int slot, int idx) {
    const bool b_side = idx >= 4;
    const int q = idx & 3;
    half_t* dst = smem + slot * STAGE_HALVES + (b_side ? kTile * BK : 0) + (q * 4 + wave) * 16 * BK;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(b_side ? b_rsrc : a_rsrc, (lds_ptr)(dst), 16,
                                             b_side ? b_off[q] : a_off[q],
                                             (k_first + kt) * (b_side ? Nb : Mb) * kSlab * 2, 0, 0);
  };
#define FASTMM_READ(kSlotSrc, kSet, r)                                                              \
  do {                                                                                              \
    if constexpr ((r) < 8)                                                                          \
      asm volatile("ds_read_b128 %0, %1 offset:%2"                                                  \
                   : "+v"(fa[kSet][(r)])                                                            \
                   : "v"(base_a[(kSlotSrc) / 2]), "i"((((kSlotSrc) % 2) * STAGE_HALVES + (r) * 16 * BK) * 2)); \
    else                                                                                            \
      asm volatile("ds_read_b128 %0, %1 offset:%2"                                                  \
                   : "+v"(fb[kSet][(r) - 8])                                                        \
                   : "v"(base_b[(kSlotSrc) / 2]),                                                   \
                     "i"((((kSlotSrc) % 2) * STAGE_HALVES + ((r) - 8) * 16 * BK) * 2));             \
  } while (0)
#define FASTMM_MFMA(kSet, q)                                                                        \
  do {                                                                                              \
    if constexpr (kIn == kBF16)                                                                     \
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"                                        \
                   : "+a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
    else                                                                                            \
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"                                         \
                   : "+a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
  } while (0)
  // 4 MFMAs with one fragment read for the next slice; a refill after every other group
#define FASTMM_GROUP(g)                                                                             \
  do {                                                                                              \
    FASTMM_MFMA(kSet, 4 * (g));                                                                     \
    FASTMM_MFMA(kSet, 4 * (g) + 1);                                                                 \
    if constexpr (kNext) FASTMM_READ(kNextSlot, 1 - kSet, (g));                                     \
    FASTMM_MFMA(kSet, 4 * (g) + 2);                                                                 \
    FASTMM_MFMA(kSet, 4 * (g) + 3);                                                                 \
    if constexpr (kLoad && (g) % 2 == 1) load_one(kt + 4, kSlot, (g) / 2);                          \
  } while (0)
#define FASTMM_TIE(i)                                                                               \
  asm volatile("" : "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3]),             \
                    "+a"(acc[i][4]), "+a"(acc[i][5]), "+a"(acc[i][6]), "+a"(acc[i][7]))
  // The compiler cannot see that an asm MFMA's result is still in flight, so an
  // accumulator copy, spill or read it places right after one would see a stale
  // value. A fence waits out the MFMA latency (24 wait states) and then claims
  // to modify every accumulator, so no compiler access to them can move above
  // it; fences close every main-loop iteration (where the allocator places loop
  // exit and back-edge copies), every tail step and the K loop.
  auto fence = [&]() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    FASTMM_TIE(0); FASTMM_TIE(1); FASTMM_TIE(2); FASTMM_TIE(3);
    FASTMM_TIE(4); FASTMM_TIE(5); FASTMM_TIE(6); FASTMM_TIE(7);
  };

  // Slice kt in ring slot kSlot, fragments in register set kSlot % 2.
  // kLoad: slice kt + 4 exists; kNext: slice kt + 1 exists; kSync: slice kt + 2
  // exists and must be resident before the barrier, with kWait loads (those of
  // slices kt + 3 and kt + 4) allowed in flight.
  auto step = [&](int kt, auto slot_tag, auto load_tag, auto next_tag, auto sync_tag, auto wait_tag) {
    constexpr int kSlot = decltype(slot_tag)::value;
    constexpr bool kLoad = decltype(load_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value;
    constexpr bool kSync = decltype(sync_tag)::value;
    constexpr int kWait = decltype(wait_tag)::value;
    constexpr int kSet = kSlot % 2, kNextSlot = (kSlot + 1) % STAGES;
    FASTMM_GROUP(0); FASTMM_GROUP(1); FASTMM_GROUP(2); FASTMM_GROUP(3);
    FASTMM_GROUP(4); FASTMM_GROUP(5); FASTMM_GROUP(6); FASTMM_GROUP(7);
    FASTMM_GROUP(8); FASTMM_GROUP(9); FASTMM_GROUP(10); FASTMM_GROUP(11);
    FASTMM_GROUP(12); FASTMM_GROUP(13); FASTMM_GROUP(14); FASTMM_GROUP(15);
    if constexpr (kSync) wait_vmcnt<kWait>();
    if constexpr (kNext) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (kSync) fast::barrier();
  };

#pragma unroll
  for (int s = 0; s < STAGES; ++s)
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) load_one(s, s, idx);
  wait_vmcnt<16>();  // slices 0 and 1 resident
  fast::barrier();
  {
    constexpr int kSrc = 0, kDst = 0;
    FASTMM_READ(kSrc, kDst, 0); FASTMM_READ(kSrc, kDst, 1); FASTMM_READ(kSrc, kDst, 2); FASTMM_READ(kSrc, kDst, 3);
    FASTMM_READ(kSrc, kDst, 4); FASTMM_READ(kSrc, kDst, 5); FASTMM_READ(kSrc, kDst, 6); FASTMM_READ(kSrc, kDst, 7);
    FASTMM_READ(kSrc, kDst, 8); FASTMM_READ(kSrc, kDst, 9); FASTMM_READ(kSrc, kDst, 10); FASTMM_READ(kSrc, kDst, 11);
    FASTMM_READ(kSrc, kDst, 12); FASTMM_READ(kSrc, kDst, 13); FASTMM_READ(kSrc, kDst, 14); FASTMM_READ(kSrc, kDst, 15);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  fast::barrier();  // every wave holds slice 0: slot 0 may be refilled
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // accumulator writes before the first MFMA
  int kt = 0;
  for (; kt < nk - 4; kt += 4) {
    step(kt, Int<0>{}, Bool<true>{}, Bool<true>{}, Bool<true>{}, Int<16>{});
    step(kt + 1, Int<1>{}, Bool<true>{}, Bool<true>{}, Bool<true>{}, Int<16>{});
    step(kt + 2, Int<2>{}, Bool<true>{}, Bool<true>{}, Bool<true>{}, Int<16>{});
    step(kt + 3, Int<3>{}, Bool<true>{}, Bool<true>{}, Bool<true>{}, Int<16>{});
    fence();
  }
  step(kt, Int<0>{}, Bool<false>{}, Bool<true>{}, Bool<true>{}, Int<8>{});
  fence();
  step(kt + 1, Int<1>{}, Bool<false>{}, Bool<true>{}, Bool<true>{}, Int<0>{});
  fence();
  step(kt + 2, Int<2>{}, Bool<false>{}, Bool<true>{}, Bool<false>{}, Int<0>{});
  fence();
  step(kt + 3, Int<3>{}, Bool<false>{}, Bool<false>{}, Bool<false>{}, Int<0>{});
  fence();
#undef FASTMM_READ
#undef FASTMM_MFMA
#undef FASTMM_GROUP
#undef FASTMM_TIE

  const int64_t leaf_offset = static_cast<int64_t>(leaf) * Mb * Nb;
  // The lane index is recomputed here (every lane is active): kept from the
  // kernel's start, the row and column bases below would be live across the K
  // loop and push accumulators into scratch memory.
  int lane_now;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_now));
  const int out_row = wm * 128 + (lane_now & 15), out_col = wn * 128 + 4 * (lane_now >> 4);
  if constexpr (kPartial) {
    float* tile_at = static_cast<float*>(P) + static_cast<int64_t>(tile_slot) * kTile * kTile;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        *reinterpret_cast<float4*>(tile_at + (out_row + i * 16) * kTile + out_col + j * 16) =
            make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      }
    }
  } else if constexpr (kOut == kFP32) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = m0 + out_row + i * 16;
      if (row >= Mb) continue;
      float* out_at = static_cast<float*>(P) + leaf_offset + static_cast<int64_t>(row) * Nb;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = n0 + out_col + j * 16;
        if (col < Nb) {
          *reinterpret_cast<float4*>(out_at + col) =
              make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        }
      }
    }
  } else {
    // Stage the 256 x 256 16-bit tile in LDS (8-byte writes: 32 lanes cover all
    // 64 banks at row pitch 264 halves), then store 16-byte row segments.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    uint16_t* staged = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = out_row + i * 16;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = out_col + j * 16;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = from_f32<kOut>(acc[i][j][e]);
        store16<4>(staged + row * fast::OUT_PITCH + col, h);
      }
    }
    __syncthreads();
    const int chunk = tid & 31;
    uint16_t* out = static_cast<uint16_t*>(P) + leaf_offset;
#pragma unroll 4
    for (int pass = 0; pass < kTile / 8; ++pass) {
      const int row = pass * 8 + (tid >> 5);
      const int grow = m0 + row, gcol = n0 + chunk * 8;
      if (grow < Mb && gcol < Nb) {
        uint16_t h[8];
        load16<8>(staged + row * fast::OUT_PITCH + chunk * 8, h);
        store16<8>(out + static_cast<int64_t>(grow) * Nb + gcol, h);
      }
    }
  }
}


// Persistent variant for 16-bit products (Kb >= 256): gridDim.x workgroups
// (a multiple of 8, one per CU) walk the tiles of their XCD's range (the same
// range decode_tile gives), gridDim.x / 8 tiles apart. One continuous slice
// stream: in a tile's last four slices the refills already fetch the next
// tile's first four, so a tile starts without waiting for memory. The output
// leaves through a 32 KB staging area after the 128 KB ring: each wave stages
// its own 128 x 128 quadrant through a private 8 KB slice (16-byte chunks
// XOR-swizzled by row: conflict-free 8-byte writes), 32 rows at a time, and
// stores 4 rows x 256 bytes per instruction (rows or columns past the leaf get
// an out-of-range offset and write nothing). A wave whose quadrant lies wholly
// past the leaf reads zeros for both MFMA operands (see set_loads), so its
// unstored products cost little power. Every wait leaves at most two steps of loads in
// flight and nothing else: vmcnt counts stores as well, and a store can
// complete before older loads (one past the buffer completes at once), so a
// wait that allowed a tile's stores in flight would not prove that the loads
// it waits for have landed. A tile's stores therefore drain during the next
// tile's first slice.
//
// kStrip fuses a last partial tile row of at most 16 rows (the "strip", rows
// tiles_m * 256 .. Mb - 1) into the tiles of the last group of 8 tile rows,
// while their B' slices are in LDS: a separate pass over the strip would
// re-read all of B' from memory. Tile (tm, tn) at position p = tm - (first
// row of the group) gives wave w the strip's 16-column block b = 4 p + w of
// tile column tn (b >= 16 or past Nb: no work). Per slice each wave issues one
// more MFMA (B' rows 16 b .. 16 b + 15 of the tile, read from LDS, against
// the strip's A' rows), one more LDS fragment read and one more load (the
// strip's A' fragment, straight into registers, four slices ahead like the
// ring); waves without work run the MFMA on zeros and store nothing. Per tile
// each wave issues one more (8-byte) store. So every step has 9 loads, and
// the waits scale to match.
constexpr int RING_BYTES = STAGES * STAGE_HALVES * 2;                      // 128 KB
constexpr int STAGE_ROWS = 64;
constexpr int PERSISTENT_LDS_BYTES = RING_BYTES + STAGE_ROWS * kTile * 2;  // 160 KB

// Cache-policy operand of the product stores when kStreamOut is set: the
// non-temporal bit (nt, bit 1 on gfx950), so products that cannot stay cached
// until the recombination reads them do not displace operand lines.
constexpr int kStoreNonTemporal = 2;

// Persistent workgroup wg of `grid` (a multiple of 8): tiles first,
// first + stride, ... (count of them) of its XCD's range, stride = grid / 8.
__device__ __forceinline__ void persistent_tiles(int wg, int grid, int total, int& first, int& stride,
                                                 int& count) {
  int start, tiles;
  xcd_range(total, wg % kXcds, start, tiles);
  const int j = wg / kXcds;
  stride = grid / kXcds;
  first = start + j;
  count = j < tiles ? (tiles - j + stride - 1) / stride : 0;
}

typedef unsigned uint4v __attribute__((ext_vector_type(4)));
typedef unsigned uint2v __attribute__((ext_vector_type(2)));

// Two values rounded to the 16-bit product type, packed (first in the low
// half). FP16 uses the packed conversion (round to nearest even, as the
// scalar one); BF16 the shared rounding helper.
template <int kOut>
__device__ __forceinline__ unsigned pack2(float lo, float hi) {
  if constexpr (kOut == kFP16) {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const half2v v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(unsigned, v);
  } else {
    return static_cast<unsigned>(from_f32<kOut>(lo)) | (static_cast<unsigned>(from_f32<kOut>(hi)) << 16);
  }
}

template <int kIn, int kOut, bool kStreamOut, bool kStrip>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void persistent_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B, uint16_t* __restrict__ P,
                       int Mb, int Nb, int Kb, int tiles_m, int tiles_n, int total_tiles) {
  extern __shared__ __attribute__((aligned(16))) half_t smem[];
  int first, stride, count;
  persistent_tiles(blockIdx.x, gridDim.x, total_tiles, first, stride, count);
  if (count == 0) return;
  const int nk = Kb / BK;  // a multiple of 4, at least 8 (checked by the launcher)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // vmcnt bound of every wait: two steps of loads in flight (the ones of the
  // slices three and four ahead), so every older load has landed
  constexpr int kLoadsPerStep = kStrip ? 9 : 8;
  constexpr int kWaitLoads = 2 * kLoadsPerStep;
  // the strip's first tile row of the last group, and the strip block of this
  // wave in tile row tm (>= 16: none)
  const int strip_group = 8 * ((tiles_m - 1) / 8);
  auto strip_block = [&](int tm) __attribute__((always_inline)) {
    return tm >= strip_group ? 4 * (tm - strip_group) + wave : 16;
  };

  // Load descriptor of the tile whose slices are being fetched (as in
  // leaf_gemm_kernel; logical < 0: no tile, every lane out of range, so the
  // loads read nothing and zero-fill their ring slots).
  constexpr unsigned kOutOfRange = 0x80000000u;
  constexpr unsigned kSegmentBytes = 64 * kSlab * 2;
  const unsigned lane_base =
      static_cast<unsigned>(((wave * 16 + (lane >> 2)) * kSlab + ((lane & 3) ^ ((lane >> 4) & 3)) * 8) * 2);
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  unsigned a_off[SEGMENTS], b_off[SEGMENTS];
  unsigned r_off = kOutOfRange;  // the strip's A' fragment (kStrip)
  // Fragment-read redirect for the descriptor's tile (bytes, uniform). A wave
  // whose 128 x 128 quadrant lies wholly past the leaf stores nothing, yet its
  // MFMAs would multiply real rows by zero-filled ones at nearly the power of
  // real work, and the leaf GEMM runs at the board's power limit. Such a wave
  // reads both operands from its zero-filled quadrant instead (A' fragments
  // from the zero B' rows past Nb, or B' fragments from the zero A' rows past
  // Mb), so its MFMAs multiply zeros: the same instructions, waits and
  // barriers, far less power. The other waves' products are unchanged.
  int load_da = 0, load_db = 0;
  auto set_loads = [&](int logical) __attribute__((always_inline)) {
    const bool none = logical < 0;
    int leaf, tm, tn;
    tile_of(none ? 0 : logical, tiles_m, tiles_n, 8, leaf, tm, tn);
    {
      const int a_quadrant = wm * 128 * BK, b_quadrant = kTile * BK + wn * 128 * BK;  // halves into a slot
      const bool past_columns = tn * kTile + wn * 128 >= Nb, past_rows = tm * kTile + wm * 128 >= Mb;
      load_da = __builtin_amdgcn_readfirstlane(past_columns ? 2 * (b_quadrant - a_quadrant) : 0);
      load_db = __builtin_amdgcn_readfirstlane(!past_columns && past_rows ? 2 * (a_quadrant - b_quadrant) : 0);
    }
    a_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(A + static_cast<int64_t>(leaf) * Mb * Kb), 0,
                                               Mb * Kb * 2, 0x00020000);
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(B + static_cast<int64_t>(leaf) * Nb * Kb), 0,
                                               Nb * Kb * 2, 0x00020000);
    const unsigned a_limit = none ? 0u : static_cast<unsigned>(Mb * kSlab * 2);
    const unsigned b_limit = none ? 0u : static_cast<unsigned>(Nb * kSlab * 2);
    const unsigned a_first = lane_base + static_cast<unsigned>(tm * kTile * kSlab * 2);
    const unsigned b_first = lane_base + static_cast<unsigned>(tn * kTile * kSlab * 2);
#pragma unroll
    for (int q = 0; q < SEGMENTS; ++q) {
      const unsigned a = a_first + q * kSegmentBytes, b = b_first + q * kSegmentBytes;
      a_off[q] = a < a_limit ? a : kOutOfRange;
      b_off[q] = b < b_limit ? b : kOutOfRange;
    }
    if constexpr (kStrip) {
      // this wave's strip A' fragment: row tiles_m * 256 + lane % 16, 8-wide K
      // chunk lane / 16 of each slab (rows past the leaf, or no block: zeros)
      const int block = strip_block(tm);
      const int row = tiles_m * kTile + (lane & 15);
      const bool active = !none && block < 16 && tn * kTile + 16 * block < Nb && row < Mb;
      r_off = active ? static_cast<unsigned>((row * kSlab + (lane >> 4) * 8) * 2) : kOutOfRange;
    }
  };

  const int fr = lane & 15, fc = lane >> 4;
  const int rd = fr * BK + ((fc ^ ((fr >> 2) & 3)) << 3);
  unsigned base_a[2], base_b[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    base_a[h] = (unsigned)(uintptr_t)(lds_ptr)(smem + h * 2 * STAGE_HALVES + wm * 128 * BK + rd);
    base_b[h] = (unsigned)(uintptr_t)(lds_ptr)(smem + h * 2 * STAGE_HALVES + kTile * BK + wn * 128 * BK + rd);
  }
  // Moves the fragment bases to the descriptor's tile's redirect: called right
  // before a tile's first fragment reads, after the previous tile's last ones.
  int applied_da = 0, applied_db = 0;
  auto redirect_reads = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      base_a[h] += static_cast<unsigned>(load_da - applied_da);
      base_b[h] += static_cast<unsigned>(load_db - applied_db);
    }
    applied_da = load_da;
    applied_db = load_db;
  };

  half8 fa[2][FM], fb[2][FN];
  float4v acc[FM][FN];  // never zeroed: a tile's first MFMAs take srcC = 0
  // kStrip: the strip block's B' fragment (a set per slice parity, from LDS),
  // the strip A' fragments (a ring of four slices, from memory) and the
  // strip's accumulator (VGPRs; the AGPRs hold acc)
  half8 fx[2] = {half8{}, half8{}};
  uint4v rfrag[STAGES] = {};
  float4v acc_x = {};
  unsigned base_x[2] = {0u, 0u};
  // base_x for the tile being computed: LDS rows 16 b + fr of its B' tile
  // (the B' fragment reads' swizzle; no block: block 15, read and unused)
  auto set_strip = [&](int logical) __attribute__((always_inline)) {
    if constexpr (kStrip) {
      int leaf, tm, tn;
      tile_of(logical, tiles_m, tiles_n, 8, leaf, tm, tn);
      const int block = min(strip_block(tm), 15);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        base_x[h] = (unsigned)(uintptr_t)(lds_ptr)(smem + h * 2 * STAGE_HALVES + kTile * BK + block * 16 * BK + rd);
      }
    }
  };
  // the strip A' fragment of slice kt of the descriptor's tile into ring slot `slot`
  auto strip_load = [&](int kt, int slot) __attribute__((always_inline)) {
    rfrag[slot] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, r_off, kt * Mb * kSlab * 2, 0);
  };
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      fa[s][i] = half8{};
      fb[s][i] = half8{};
    }

  // idx 0..3: A' segments, 4..7: B' segments of slice kt of the descriptor's tile
  auto load_one = [&](int kt, int slot, int idx) __attribute__((always_inline)) {
    const bool b_side = idx >= 4;
    const int q = idx & 3;
    half_t* dst = smem + slot * STAGE_HALVES + (b_side ? kTile * BK : 0) + (q * 4 + wave) * 16 * BK;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(b_side ? b_rsrc : a_rsrc, (lds_ptr)(dst), 16,
                                             b_side ? b_off[q] : a_off[q], kt * (b_side ? Nb : Mb) * kSlab * 2,
                                             0, 0);
  };
#define FASTMM_READ(kSlotSrc, kSet, r)                                                              \
  do {                                                                                              \
    if constexpr ((r) < 8)                                                                          \
      asm volatile("ds_read_b128 %0, %1 offset:%2"                                                  \
                   : "+v"(fa[kSet][(r)])                                                            \
                   : "v"(base_a[(kSlotSrc) / 2]), "i"((((kSlotSrc) % 2) * STAGE_HALVES + (r) * 16 * BK) * 2)); \
    else                                                                                            \
      asm volatile("ds_read_b128 %0, %1 offset:%2"                                                  \
                   : "+v"(fb[kSet][(r) - 8])                                                        \
                   : "v"(base_b[(kSlotSrc) / 2]),                                                   \
                     "i"((((kSlotSrc) % 2) * STAGE_HALVES + ((r) - 8) * 16 * BK) * 2));             \
  } while (0)
#define FASTMM_MFMA(kSet, q)                                                                        \
  do {                                                                                              \
    if constexpr (kFirst && kIn == kBF16)                                                           \
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"                                         \
                   : "=a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
    else if constexpr (kFirst)                                                                      \
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0"                                          \
                   : "=a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
    else if constexpr (kIn == kBF16)                                                                \
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"                                        \
                   : "+a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
    else                                                                                            \
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"                                         \
                   : "+a"(acc[(q) / 8][(q) % 8])                                                    \
                   : "v"(fb[kSet][(q) % 8]), "v"(fa[kSet][(q) / 8]));                               \
  } while (0)
#define FASTMM_GROUP(g)                                                                             \
  do {                                                                                              \
    FASTMM_MFMA(kSet, 4 * (g));                                                                     \
    FASTMM_MFMA(kSet, 4 * (g) + 1);                                                                 \
    if constexpr (kNext) FASTMM_READ(kNextSlot, 1 - kSet, (g));                                     \
    FASTMM_MFMA(kSet, 4 * (g) + 2);                                                                 \
    FASTMM_MFMA(kSet, 4 * (g) + 3);                                                                 \
    if constexpr (kLoad && (g) % 2 == 1) load_one(load_kt, kSlot, (g) / 2);                         \
  } while (0)
#define FASTMM_TIE(i)                                                                               \
  asm volatile("" : "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3]),             \
                    "+a"(acc[i][4]), "+a"(acc[i][5]), "+a"(acc[i][6]), "+a"(acc[i][7]))
  // The strip MFMA accumulates in VGPRs (early clobber on the first: its
  // destination must not overlap the sources).
#define FASTMM_STRIP_MFMA(kSet, kSlot)                                                              \
  do {                                                                                              \
    if constexpr (kFirst && kIn == kBF16)                                                           \
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"                                         \
                   : "=&v"(acc_x) : "v"(fx[kSet]), "v"(rfrag[kSlot]));                              \
    else if constexpr (kFirst)                                                                      \
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0"                                          \
                   : "=&v"(acc_x) : "v"(fx[kSet]), "v"(rfrag[kSlot]));                              \
    else if constexpr (kIn == kBF16)                                                                \
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"                                        \
                   : "+v"(acc_x) : "v"(fx[kSet]), "v"(rfrag[kSlot]));                               \
    else                                                                                            \
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"                                         \
                   : "+v"(acc_x) : "v"(fx[kSet]), "v"(rfrag[kSlot]));                               \
  } while (0)
#define FASTMM_STRIP_READ(kSlotSrc, kSet)                                                           \
  asm volatile("ds_read_b128 %0, %1 offset:%2"                                                      \
               : "+v"(fx[kSet])                                                                     \
               : "v"(base_x[(kSlotSrc) / 2]), "i"(((kSlotSrc) % 2) * STAGE_HALVES * 2))
  auto fence = [&]() __attribute__((always_inline)) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    FASTMM_TIE(0); FASTMM_TIE(1); FASTMM_TIE(2); FASTMM_TIE(3);
    FASTMM_TIE(4); FASTMM_TIE(5); FASTMM_TIE(6); FASTMM_TIE(7);
    if constexpr (kStrip) asm volatile("" : "+v"(acc_x));
  };

  // The vmcnt wait of every step and of the prologue (kWaitLoads in flight).
  auto wait_loads = [&]() __attribute__((always_inline)) {
    if constexpr (kWaitLoads == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if constexpr (kWaitLoads == 18) asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
    else static_assert(kWaitLoads < 0, "unsupported vmcnt");
  };
  // One slice in ring slot kSlot (fragments in register set kSlot % 2): kLoad
  // refills the slot with slice load_kt of the descriptor's tile; kNext reads
  // the next slice's fragments; the wait leaves the loads of the slices three
  // and four ahead in flight, so the slice two ahead is resident; kFirst
  // starts the accumulators.
  auto step = [&](int load_kt, auto slot_tag, auto load_tag, auto next_tag, auto first_tag)
      __attribute__((always_inline)) {
    constexpr int kSlot = decltype(slot_tag)::value;
    constexpr bool kLoad = decltype(load_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value;
    constexpr bool kFirst = decltype(first_tag)::value;
    constexpr int kSet = kSlot % 2, kNextSlot = (kSlot + 1) % STAGES;
    FASTMM_GROUP(0); FASTMM_GROUP(1); FASTMM_GROUP(2); FASTMM_GROUP(3);
    FASTMM_GROUP(4); FASTMM_GROUP(5); FASTMM_GROUP(6); FASTMM_GROUP(7);
    FASTMM_GROUP(8); FASTMM_GROUP(9); FASTMM_GROUP(10); FASTMM_GROUP(11);
    FASTMM_GROUP(12); FASTMM_GROUP(13); FASTMM_GROUP(14); FASTMM_GROUP(15);
    if constexpr (kStrip) {
      // the strip block: this slice's MFMA, then the next slice's B' fragment
      // and (after the MFMA has read it) a refill of this ring slot's A' one
      FASTMM_STRIP_MFMA(kSet, kSlot);
      if constexpr (kNext) FASTMM_STRIP_READ(kNextSlot, 1 - kSet);
      if constexpr (kLoad) strip_load(load_kt, kSlot);
    }
    wait_loads();
    if constexpr (kNext) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    fast::barrier();
  };
  // A tile's first four slices (refilled with its slices 4..7).
  auto first_group = [&]() __attribute__((always_inline)) {
    step(4, Int<0>{}, Bool<true>{}, Bool<true>{}, Bool<true>{});
    step(5, Int<1>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(6, Int<2>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(7, Int<3>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    fence();
  };
  auto steady_group = [&](int load_kt) __attribute__((always_inline)) {
    step(load_kt, Int<0>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(load_kt + 1, Int<1>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(load_kt + 2, Int<2>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(load_kt + 3, Int<3>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    fence();
  };
  // A tile's last four slices: the refills fetch slices 0..3 of the next tile
  // (the descriptor was switched), and the last step reads no fragments, so
  // both fragment sets are free in the epilogue.
  auto boundary_group = [&]() __attribute__((always_inline)) {
    step(0, Int<0>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(1, Int<1>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(2, Int<2>{}, Bool<true>{}, Bool<true>{}, Bool<false>{});
    step(3, Int<3>{}, Bool<true>{}, Bool<false>{}, Bool<false>{});
    fence();
  };
  // Slice-0 fragments (ring slot 0) into register set 0; every wave's reads
  // done before slot 0 is refilled.
  auto read_first_slice = [&]() __attribute__((always_inline)) {
    constexpr int kSrc = 0, kDst = 0;
    FASTMM_READ(kSrc, kDst, 0); FASTMM_READ(kSrc, kDst, 1); FASTMM_READ(kSrc, kDst, 2); FASTMM_READ(kSrc, kDst, 3);
    FASTMM_READ(kSrc, kDst, 4); FASTMM_READ(kSrc, kDst, 5); FASTMM_READ(kSrc, kDst, 6); FASTMM_READ(kSrc, kDst, 7);
    FASTMM_READ(kSrc, kDst, 8); FASTMM_READ(kSrc, kDst, 9); FASTMM_READ(kSrc, kDst, 10); FASTMM_READ(kSrc, kDst, 11);
    FASTMM_READ(kSrc, kDst, 12); FASTMM_READ(kSrc, kDst, 13); FASTMM_READ(kSrc, kDst, 14); FASTMM_READ(kSrc, kDst, 15);
    if constexpr (kStrip) FASTMM_STRIP_READ(kSrc, kDst);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    fast::barrier();
  };

  const unsigned stage_base = (unsigned)(uintptr_t)(lds_ptr)(smem) + RING_BYTES;
  set_loads(first);
#pragma unroll
  for (int s = 0; s < STAGES; ++s) {
#pragma unroll
    for (int idx = 0; idx < 8; ++idx) load_one(s, s, idx);
    if constexpr (kStrip) strip_load(s, s);
  }
  wait_loads();  // slices 0 and 1 resident
  fast::barrier();
  set_strip(first);
  redirect_reads();
  read_first_slice();

  for (int t = 0; t < count; ++t) {
    const int logical = first + t * stride;
    first_group();
    for (int kt = 4; kt < nk - 4; kt += 4) steady_group(kt + 4);
    set_loads(t + 1 < count ? logical + stride : -1);
    boundary_group();

    // Epilogue: each wave stages only its own 128 x 128 quadrant, in four
    // passes of 32 rows through a private 8 KB slice of the staging area, so
    // no wave waits for another. Lane (r = lane % 16, g = lane / 16) writes
    // the 4 columns 16 j + 4 g .. +3 of quadrant row 16 ii + r (8 bytes) into
    // 16-byte chunk (2 j + g / 2) ^ r of a 256-byte staging row (bytes 8 (g % 2)
    // within it): for each j the 64 lanes fill all 64 banks twice over, with no
    // conflict. It reads back 16-byte chunks (lane % 16) of rows 4 h + lane / 16
    // and stores 4 quadrant rows x 256 bytes per instruction. The tile's base
    // offset goes in the stores' scalar offset; lanes outside the leaf get an
    // offset past the buffer and write nothing.
    int leaf, tm, tn;
    tile_of(logical, tiles_m, tiles_n, 8, leaf, tm, tn);
    const unsigned m0 = tm * kTile + wm * 128, n0 = tn * kTile + wn * 128;  // quadrant origin
    const __amdgpu_buffer_rsrc_t p_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        P + static_cast<int64_t>(leaf) * Mb * Nb, 0, Mb * Nb * 2, 0x00020000);
    // lane recomputed here (every lane is active), so no lane-derived value
    // stays live across the K loop
    int lane_now;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_now));
    const unsigned er = lane_now & 15, eg = lane_now >> 4;
    const unsigned wave_stage = stage_base + static_cast<unsigned>(wave) * (32 * 256);
    unsigned write_at[FN], read_at[4];
#pragma unroll
    for (int j = 0; j < FN; ++j) write_at[j] = wave_stage + er * 256 + (((2 * j + (eg >> 1)) ^ er) << 4) + ((eg & 1) << 3);
#pragma unroll
    for (int h = 0; h < 4; ++h) read_at[h] = wave_stage + (4 * h + eg) * 256 + ((er ^ ((4 * h + eg) & 15)) << 4);
    const unsigned nb_u = static_cast<unsigned>(Nb);
    const unsigned lane_offset = (eg * nb_u + er * 8) * 2;  // row eg, column 8 er of a 4-row store
    const unsigned mb_u = static_cast<unsigned>(Mb);
    const bool column_inside = n0 + er * 8 < nb_u;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = 2 * c + ii;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const uint2v v = {pack2<kOut>(acc[i][j][0], acc[i][j][1]), pack2<kOut>(acc[i][j][2], acc[i][j][3])};
          asm volatile("ds_write_b64 %0, %1 offset:%2" : : "v"(write_at[j]), "v"(v), "i"(ii * 16 * 256) : "memory");
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      uint4v staged[8];
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(staged[h]) : "v"(read_at[h & 3]), "i"((h >> 2) * 16 * 256)
                     : "memory");
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        const unsigned row0 = m0 + 32 * c + 4 * h;  // first of the instruction's 4 rows (uniform)
        const bool inside = (row0 + eg < mb_u) && column_inside;
        // a base past the leaf is zeroed so that the out-of-range offset cannot
        // wrap into the buffer (in-range bases stay below Mb * Nb * 2 <= 2^31 - 1,
        // which the launcher checks)
        const unsigned base = (row0 < mb_u && n0 < nb_u) ? (row0 * nb_u + n0) * 2 : 0u;
        __builtin_amdgcn_raw_buffer_store_b128(staged[h], p_rsrc, inside ? lane_offset : kOutOfRange,
                                               static_cast<int>(base), kStreamOut ? kStoreNonTemporal : 0);
      }
      asm volatile("" ::: "memory");
    }
    if constexpr (kStrip) {
      // this wave's strip block: lane l holds row tiles_m * 256 + l % 16,
      // columns 16 b + 4 (l / 16) .. + 3 of the tile (8 bytes)
      const int block = strip_block(tm);
      const unsigned row = static_cast<unsigned>(tiles_m * kTile) + er;
      const unsigned col = tn * kTile + 16 * static_cast<unsigned>(block) + 4 * eg;
      const bool inside = block < 16 && row < mb_u && col < nb_u;  // Nb % 8 == 0: all 4 columns or none
      const uint2v v = {pack2<kOut>(acc_x[0], acc_x[1]), pack2<kOut>(acc_x[2], acc_x[3])};
      __builtin_amdgcn_raw_buffer_store_b64(v, p_rsrc, inside ? (row * nb_u + col) * 2 : kOutOfRange, 0,
                                            kStreamOut ? kStoreNonTemporal : 0);
      asm volatile("" ::: "memory");
      if (t + 1 < count) set_strip(logical + stride);
    }
    redirect_reads();  // the descriptor now holds the next tile
    read_first_slice();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (empty) refills have landed in LDS
#undef FASTMM_READ
#undef FASTMM_MFMA
#undef FASTMM_GROUP
#undef FASTMM_TIE
#undef FASTMM_STRIP_MFMA
#undef FASTMM_STRIP_READ
}

}  // namespace mfma16

// ------------------------------------------------------- thin last tile row

// When a leaf's last row of 256x256 tiles holds at most 16 rows (Mb % 256 in
// 1..16, e.g. Mb = 4107), those tiles would run a whole tile's MFMAs for a few
// rows and, in count, push the tiles past a round boundary (at Mb = 4107:
// 1071 tiles, 47 past four rounds). They run here instead, as one 16-row
// block: tiles of 64 columns (grid: column tiles x leaves), each wave 16
// columns, operands straight from the K-slab planes into registers (16-byte
// loads, four slices in flight). The strip reads all of B' once, so it pays
// off only for a few rows and a small B' (leaf_plan decides). Each product is the same v_mfma_f32_16x16x32
// sequence over the same 32-wide K slices, in the same operand order, as in
// the 256 x 256 kernels, so the products are bit-identical.
namespace thin {

constexpr int kRows = 16, kCols = 64;
using mfma16::uint4v;

template <int kIn>
__device__ __forceinline__ float4v mfma_16x16x32(uint4v a, uint4v b, float4v c) {
  if constexpr (kIn == kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                   0, 0);
  }
}

template <int kIn, int kOut>
__global__ __launch_bounds__(kGemmThreads) void thin_rows_kernel(const half_t* __restrict__ A,
                                                                 const half_t* __restrict__ B, void* __restrict__ P,
                                                                 int Mb, int Nb, int Kb, int m0) {
  const int leaf = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int fr = lane & 15, fk = lane >> 4;  // fragment row, 8-wide K chunk
  // Fragment addresses in slab 0 of the leaf's planes. Rows or columns past
  // the leaf read a clamped valid element: their products only reach output
  // rows or columns that are not stored (row m of P needs only row m of A',
  // column n only row n of B').
  const half_t* a_base =
      A + static_cast<int64_t>(leaf) * Mb * Kb + min(m0 + fr, Mb - 1) * kSlab + fk * 8;
  const int col = blockIdx.x * kCols + wave * 16 + fr;
  const half_t* b_base = B + static_cast<int64_t>(leaf) * Nb * Kb + min(col, Nb - 1) * kSlab + fk * 8;
  // kDepth slices of fragments in flight, a ring of registers (nk is a
  // multiple of 4 on this path; refills past the last slice re-read it). The
  // loads are asm with explicit waits: compiler-placed waits at the loop head
  // would drain the whole ring every iteration.
  constexpr int kDepth = 4;
  const int nk = Kb / kSlab;
  uint4v bf[kDepth], af[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) bf[d] = af[d] = uint4v{0, 0, 0, 0};
  auto fetch = [&](int slot, int kt) __attribute__((always_inline)) {
    kt = kt < nk ? kt : nk - 1;
    asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(bf[slot]) : "v"(b_base + static_cast<int64_t>(kt) * Nb * kSlab));
    asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(af[slot]) : "v"(a_base + static_cast<int64_t>(kt) * Mb * kSlab));
  };
#pragma unroll
  for (int d = 0; d < kDepth; ++d) fetch(d, d);
  float4v acc = {};
  for (int kt = 0; kt < nk; kt += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      // slot d landed, the other three slots' six loads may be in flight; the
      // slot's registers are tied so the MFMA cannot move above the wait
      static_assert(kDepth == 4, "vmcnt below is (kDepth - 1) * 2");
      asm volatile("s_waitcnt vmcnt(6)" : "+v"(bf[d]), "+v"(af[d]) : : "memory");
      acc = mfma_16x16x32<kIn>(bf[d], af[d], acc);  // operands (B', A'): lane l holds row l%16
      fetch(d, kt + d + kDepth);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // element e of lane l: row m0 + l%16, column (16-column block) + 4*(l/16) + e
  const int row = m0 + fr, out_col = blockIdx.x * kCols + wave * 16 + 4 * fk;
  if (row >= Mb || out_col >= Nb) return;
  const int64_t at = static_cast<int64_t>(leaf) * Mb * Nb + static_cast<int64_t>(row) * Nb + out_col;
  if constexpr (kOut == kFP32) {
    *reinterpret_cast<float4*>(static_cast<float*>(P) + at) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  } else {
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = from_f32<kOut>(acc[e]);
    store16<4>(static_cast<uint16_t*>(P) + at, h);
  }
}

}  // namespace thin

// -------------------------------------------------------------- generic path

namespace generic {

constexpr int BK = 64;
constexpr int A_CHUNKS = kTile * BK / 8 / kGemmThreads;
constexpr int STAGE_HALVES = 2 * kTile * BK;
constexpr int LDS_BYTES = 2 * STAGE_HALVES * 2;

// Chunk c (8 halves) of row r at c ^ (r & 7).
__device__ __forceinline__ int swizzled(int row, int chunk) {
  return row * BK + ((chunk ^ (row & 7)) << 3);
}

// kSlabLayout: operand planes are K-slab-major (Kb % 32 == 0); a thread's 8
// consecutive k stay inside one slab row.
template <bool kAligned, int kIn, int kOut, bool kSlabLayout>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void leaf_gemm_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                      void* __restrict__ P, int Mb, int Nb, int Kb, int tiles_m, int tiles_n,
                      int total_tiles) {
  constexpr int TM = 4, TN = 4;
  extern __shared__ __attribute__((aligned(16))) half_t smem[];
  int leaf, tm, tn;
  decode_tile(blockIdx.x, total_tiles, tiles_m, tiles_n, 4, leaf, tm, tn);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = tm * kTile, n0 = tn * kTile;
  const half_t* a_leaf = A + static_cast<int64_t>(leaf) * Mb * Kb;
  const half_t* b_leaf = B + static_cast<int64_t>(leaf) * Nb * Kb;

  uint4 a_regs[A_CHUNKS], b_regs[A_CHUNKS];
  auto load_rows = [&](const half_t* base, int row0, int rows, int k0, uint4* regs) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int id = i * kGemmThreads + tid;
      const int grow = row0 + (id >> 3);
      const int k = k0 + ((id & 7) << 3);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (grow < rows) {
        const half_t* p = base + operand_offset<kSlabLayout>(grow, k, rows, Kb);
        if constexpr (kAligned) {
          if (k < Kb) v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = (k + e < Kb) ? __builtin_bit_cast(uint16_t, p[e]) : uint16_t{0};
          __builtin_memcpy(&v, h, 16);
        }
      }
      regs[i] = v;
    }
  };
  auto lds_store = [&](int buffer) {
    half_t* as = smem + buffer * STAGE_HALVES;
    half_t* bs = as + kTile * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int id = i * kGemmThreads + tid;
      *reinterpret_cast<uint4*>(as + swizzled(id >> 3, id & 7)) = a_regs[i];
      *reinterpret_cast<uint4*>(bs + swizzled(id >> 3, id & 7)) = b_regs[i];
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int k_tiles = (Kb + BK - 1) / BK;
  load_rows(a_leaf, m0, Mb, 0, a_regs);
  load_rows(b_leaf, n0, Nb, 0, b_regs);
  lds_store(0);
  __syncthreads();
  const int lane_row = lane & 31, lane_half = lane >> 5;
  for (int kt = 0; kt < k_tiles; ++kt) {
    const int buffer = kt & 1;
    if (kt + 1 < k_tiles) {
      load_rows(a_leaf, m0, Mb, (kt + 1) * BK, a_regs);
      load_rows(b_leaf, n0, Nb, (kt + 1) * BK, b_regs);
    }
    const half_t* as = smem + buffer * STAGE_HALVES;
    const half_t* bs = as + kTile * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = 2 * ks + lane_half;
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const half8*>(as + swizzled(wm * 128 + i * 32 + lane_row, chunk));
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const half8*>(bs + swizzled(wn * 128 + j * 32 + lane_row, chunk));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = mfma_32x32x16<kIn>(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < k_tiles) lds_store(buffer ^ 1);
    __syncthreads();
  }

  // lane l, element e of accumulator (i, j): row 8*(e/4) + 4*(l/32) + e%4,
  // column l%32 of that 32x32 block.
  const int64_t leaf_offset = static_cast<int64_t>(leaf) * Mb * Nb;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * 128 + j * 32 + lane_row;
      if (col >= Nb) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * lane_half + (e & 3);
        if (row < Mb) {
          const int64_t offset = leaf_offset + static_cast<int64_t>(row) * Nb + col;
          if constexpr (kOut == kFP32) static_cast<float*>(P)[offset] = acc[i][j][e];
          else static_cast<uint16_t*>(P)[offset] = from_f32<kOut>(acc[i][j][e]);
        }
      }
    }
}

}  // namespace generic

// ------------------------------------------------------------- split-K tail

// Sum of the `split` fp32 parts of each tail tile, in K order, cast to the
// products type and stored inside the leaf (rows < Mb, columns < Nb). A thread
// owns 4 consecutive columns of one tile row; Nb % 4 == 0 (checked by the
// launcher), so the 4 are all inside or all outside.
template <int kOut>
__global__ __launch_bounds__(256) void tail_reduce_kernel(const float* __restrict__ partial, void* __restrict__ P,
                                                          int Mb, int Nb, int tiles_m, int tiles_n, int tail_base,
                                                          int split) {
  const int t = blockIdx.y;
  const int e = (blockIdx.x * 256 + threadIdx.x) * 4;
  int leaf, tm, tn;
  tile_of(tail_base + t, tiles_m, tiles_n, 8, leaf, tm, tn);
  const int row = tm * kTile + (e / kTile), col = tn * kTile + (e % kTile);
  if (row >= Mb || col >= Nb) return;
  const float* part = partial + static_cast<int64_t>(t) * split * kTile * kTile + e;
  float4 sum = *reinterpret_cast<const float4*>(part);
  for (int p = 1; p < split; ++p) {
    const float4 v = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(p) * kTile * kTile);
    sum.x += v.x;
    sum.y += v.y;
    sum.z += v.z;
    sum.w += v.w;
  }
  const int64_t at = static_cast<int64_t>(leaf) * Mb * Nb + static_cast<int64_t>(row) * Nb + col;
  if constexpr (kOut == kFP32) {
    *reinterpret_cast<float4*>(static_cast<float*>(P) + at) = sum;
  } else {
    uint16_t h[4] = {from_f32<kOut>(sum.x), from_f32<kOut>(sum.y), from_f32<kOut>(sum.z), from_f32<kOut>(sum.w)};
    store16<4>(static_cast<uint16_t*>(P) + at, h);
  }
}


// One workgroup per CU: `total` tiles run in ceil(total / CUs) rounds, and a
// last round of `tail` < CUs tiles leaves CUs idle for a whole tile time. The
// tail's tiles are split along K into `split` parts run side by side, then
// added by tail_reduce_kernel: the last round takes ~1/split of a tile time
// plus the reduction. split = min(8, groups of 4 slices, 3/4 CUs / tail), and
// no split below 2. The 3/4 matters: a round that leaves CUs idle runs at a
// higher clock (the chip is power-limited), so on MI355X a split filling every
// CU lost ~5 % against whole tiles (tail of 128 tiles in 2 parts), while
// splits over at most 3/4 of the CUs gained 2-25 %, most for small tails.
struct TailSplit {
  int64_t main_tiles, tail, split;
};

TailSplit tail_split(int64_t total, int64_t kb) {
  const int64_t cus = compute_units();
  const int64_t groups = kb / (4 * mfma16::BK);
  if (cus <= 0) return {total, 0, 1};
  const int64_t tail = total % cus;
  if (tail == 0) return {total, 0, 1};
  const int64_t split = std::min<int64_t>({8, groups, 3 * cus / (4 * tail)});
  if (split < 2) return {total, 0, 1};
  return {total - tail, tail, split};
}

int64_t tail_scratch_bytes(const TailSplit& plan) {
  return plan.tail * plan.split * kTile * kTile * static_cast<int64_t>(sizeof(float));
}

// The 16x16x32 path's launch plan: the split-K tail is planned on the
// 256 x 256 tiles, and a last tile row of at most 16 rows (below a full one)
// is left out of them when that takes the tiles down a round. The persistent
// kernel's strip form takes it where it applies (leaf_plan): at 8214 x 12288
// x 4608 that made the leaf stage 1.8 % (rank 7) and 6.2 % (rank 48) faster
// than the paths below. Otherwise thin_rows_kernel takes it if the strip is
// cheap there: a separate pass re-reads all of B' (R * Nb * Kb * 2 bytes),
// about R * Nb / 64K tile rounds at any Kb. It saved 4 % of the leaf stage at
// R * Nb = 16128 (rank 7, 8214 x 12288 x 4608) and lost 1.4 % at 55296
// (rank 48, same shape), where the row then runs as whole tiles.
constexpr int64_t kThinMaxRankColumns = 32768;

struct LeafPlan {
  int64_t tiles_m, tiles_n;  // 256 x 256 tiles (the thin row or strip excluded)
  bool thin;   // the last (partial) tile row by thin_rows_kernel
  bool strip;  // the last (partial) tile row fused into the persistent kernel
  TailSplit split;
};

// A last tile row of at most 16 rows is left out of the tiles when that takes
// them down a round. It then goes into the persistent kernel as a strip when
// the tiles have no split-K tail and the last group of 8 tile rows has at
// least 4 (one strip block per wave and tile covers its 16 blocks); the
// launcher runs thin_rows_kernel over it when the persistent kernel is not
// used. Otherwise thin_rows_kernel takes it if the strip is cheap there.
LeafPlan leaf_plan(int64_t rank, int64_t mb, int64_t kb, int64_t nb) {
  const int64_t rem = mb % kTile, tiles_n = ceil_div(nb, kTile);
  const int64_t with_row = ceil_div(mb, kTile) * tiles_n * rank, without_row = with_row - tiles_n * rank;
  const int64_t cus = compute_units();
  const bool drop = mb > kTile && rem > 0 && rem <= thin::kRows && cus > 0 &&
                    ceil_div(without_row, cus) < ceil_div(with_row, cus);
  if (drop) {
    const int64_t full = mb / kTile, last_group = full - 8 * ((full - 1) / 8);
    const TailSplit split = tail_split(without_row, kb);
    if (last_group >= 4 && split.tail == 0) return {full, tiles_n, false, true, split};
  }
  const bool thin = drop && rank * nb <= kThinMaxRankColumns;
  const int64_t tiles_m = ceil_div(mb, kTile) - (thin ? 1 : 0);
  return {tiles_m, tiles_n, thin, false, tail_split(rank * tiles_m * tiles_n, kb)};
}

// ---------------------------------------------------------------- launchers

// hipFuncSetAttribute (the dynamic LDS reservation above 64 KB) once per
// kernel and device; `devices` holds one bit per device already configured
// (atomic: first calls may race from several host threads, and setting the
// attribute twice is harmless).
template <class Kernel>
int reserve_lds(Kernel kernel, int lds_bytes, std::atomic<uint64_t>& devices) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(FASTMM_ERROR_LAUNCH, "leaf products: no current device");
  const uint64_t bit = device >= 0 && device < 64 ? uint64_t{1} << device : 0;
  if (bit != 0 && (devices.load(std::memory_order_acquire) & bit) != 0) return FASTMM_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          lds_bytes) != hipSuccess) {
    return fail(FASTMM_ERROR_LAUNCH, "leaf products: cannot reserve %d bytes of LDS", lds_bytes);
  }
  devices.fetch_or(bit, std::memory_order_release);
  return FASTMM_OK;
}

// The same reservation for an optional kernel: false when the device refuses
// it, leaving no error behind (the runtime's last error is cleared) and not
// asking that device again.
template <class Kernel>
bool try_reserve_lds(Kernel kernel, int lds_bytes, std::atomic<uint64_t>& granted,
                     std::atomic<uint64_t>& refused) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
    (void)hipGetLastError();
    return false;
  }
  const uint64_t bit = uint64_t{1} << device;
  if ((granted.load(std::memory_order_acquire) & bit) != 0) return true;
  if ((refused.load(std::memory_order_acquire) & bit) != 0) return false;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          lds_bytes) != hipSuccess) {
    (void)hipGetLastError();
    refused.fetch_or(bit, std::memory_order_release);
    return false;
  }
  granted.fetch_or(bit, std::memory_order_release);
  return true;
}

template <class Kernel>
int launch_tiles(Kernel kernel, int lds_bytes, const void* a, const void* b, void* p,
                 int64_t rank, int64_t mb, int64_t kb, int64_t nb, hipStream_t stream) {
  static std::atomic<uint64_t> configured{0};  // one per kernel instantiation
  if (int status = reserve_lds(kernel, lds_bytes, configured)) return status;
  const int64_t tiles_m = ceil_div(mb, kTile);
  const int64_t tiles_n = ceil_div(nb, kTile);
  const int64_t total = tiles_m * tiles_n * rank;
  if (total > INT32_MAX) return fail(FASTMM_ERROR_UNSUPPORTED, "leaf products: too many tiles");
  kernel<<<dim3(static_cast<unsigned>(total)), kGemmThreads, lds_bytes, stream>>>(
      static_cast<const half_t*>(a), static_cast<const half_t*>(b), p, static_cast<int>(mb),
      static_cast<int>(nb), static_cast<int>(kb), static_cast<int>(tiles_m),
      static_cast<int>(tiles_n), static_cast<int>(total));
  return check_launch("leaf products");
}

// The fast kernels' preconditions; the generic kernel handles everything else.
bool fast_leaf_gemm_applies(const void* a, const void* b, const void* p, int64_t kb, int64_t nb,
                            int products_dtype) {
  const int64_t out_align = products_dtype == kFP32 ? 4 : 8;
  return kb % fast::BK == 0 && kb >= 3 * fast::BK && nb % out_align == 0 && aligned_to(a, 16) &&
         aligned_to(b, 16) && aligned_to(p, 16);
}

// The 16x16x32 kernel additionally needs whole groups of four slices and leaf
// planes whose byte offsets fit its 32-bit buffer addressing; num_records (the
// plane's bytes) stays below 2^31, the offset it uses for padding rows.
bool mfma16_leaf_gemm_applies(int64_t mb, int64_t kb, int64_t nb) {
  return kb % (4 * mfma16::BK) == 0 && (mb + kTile) * kb * 2 <= INT32_MAX &&
         (nb + kTile) * kb * 2 <= INT32_MAX;
}

// The 16x16x32 kernel over all tiles, with the split-K tail when scratch
// holds its partial sums (otherwise the tail runs as whole tiles).
template <int kIn, int kOut>
int launch_mfma16(const void* a, const void* b, void* p, int64_t rank, int64_t mb, int64_t kb, int64_t nb,
                  void* scratch, int64_t scratch_bytes, hipStream_t stream) {
  static std::atomic<uint64_t> main_ready{0}, partial_ready{0};
  auto* main_kernel = mfma16::leaf_gemm_kernel<kIn, kOut, false>;
  auto* partial_kernel = mfma16::leaf_gemm_kernel<kIn, kFP32, true>;
  if (int status = reserve_lds(main_kernel, mfma16::LDS_BYTES, main_ready)) return status;
  if (int status = reserve_lds(partial_kernel, mfma16::LDS_BYTES, partial_ready)) return status;
  if (ceil_div(mb, kTile) * ceil_div(nb, kTile) * rank > INT32_MAX / 4) {
    return fail(FASTMM_ERROR_UNSUPPORTED, "leaf products: too many tiles");
  }
  const LeafPlan layout = leaf_plan(rank, mb, kb, nb);
  const int64_t tiles_m = layout.tiles_m, tiles_n = layout.tiles_n;
  const int64_t total = tiles_m * tiles_n * rank;
  TailSplit plan = layout.split;
  if (plan.tail > 0 && (scratch == nullptr || scratch_bytes < tail_scratch_bytes(plan) ||
                        !aligned_to(scratch, 16))) {
    plan = {total, 0, 1};
  }
  const half_t* A = static_cast<const half_t*>(a);
  const half_t* B = static_cast<const half_t*>(b);
  const int M = static_cast<int>(mb), N = static_cast<int>(nb), K = static_cast<int>(kb);
  const int TM = static_cast<int>(tiles_m), TN = static_cast<int>(tiles_n);
  // More than one round of whole tiles: the persistent kernel (16-bit
  // products, at least 8 slices, 32-bit store offsets, and the 160 KB LDS
  // reservation granted; otherwise one workgroup per tile).
  bool persistent = false;
  if constexpr (kOut != kFP32) {
    // Products beyond 1 GiB (four times the Infinity Cache) are stored with the
    // non-temporal hint. Measured on the C2-C5 leaf problems: 2.0 GB of
    // products (K = 1024) -3 % leaf time; 0.40 GB +3 %; 0.13-0.23 GB no change.
    const bool stream_out = rank * mb * nb * 2 > (int64_t{1} << 30);
    const int variant = (stream_out ? 1 : 0) + (layout.strip ? 2 : 0);
    static std::atomic<uint64_t> persistent_granted[4], persistent_refused[4];
    decltype(&mfma16::persistent_kernel<kIn, kOut, false, false>) const kernels[4] = {
                              mfma16::persistent_kernel<kIn, kOut, false, false>,
                              mfma16::persistent_kernel<kIn, kOut, true, false>,
                              mfma16::persistent_kernel<kIn, kOut, false, true>,
                              mfma16::persistent_kernel<kIn, kOut, true, true>};
    auto* kernel = kernels[variant];
    const int64_t grid = compute_units() / 8 * 8;
    persistent = grid >= 8 && plan.main_tiles > grid && kb >= 8 * mfma16::BK && mb * nb * 2 <= INT32_MAX &&
                 try_reserve_lds(kernel, mfma16::PERSISTENT_LDS_BYTES, persistent_granted[variant],
                                 persistent_refused[variant]);
    if (persistent) {
      kernel<<<dim3(static_cast<unsigned>(grid)), kGemmThreads, mfma16::PERSISTENT_LDS_BYTES, stream>>>(
          A, B, static_cast<uint16_t*>(p), M, N, K, TM, TN, static_cast<int>(plan.main_tiles));
      if (int status = check_launch("leaf products")) return status;
    }
  }
  if (!persistent && plan.main_tiles > 0) {
    main_kernel<<<dim3(static_cast<unsigned>(plan.main_tiles)), kGemmThreads, mfma16::LDS_BYTES, stream>>>(
        A, B, p, M, N, K, TM, TN, static_cast<int>(plan.main_tiles), 0, 1, 1);
    if (int status = check_launch("leaf products")) return status;
  }
  if (plan.tail > 0) {
    const int tail = static_cast<int>(plan.tail), split = static_cast<int>(plan.split);
    const int base = static_cast<int>(plan.main_tiles);
    partial_kernel<<<dim3(static_cast<unsigned>(tail * split)), kGemmThreads, mfma16::LDS_BYTES, stream>>>(
        A, B, scratch, M, N, K, TM, TN, 0, base, tail, split);
    if (int status = check_launch("leaf products (split-K tail)")) return status;
    tail_reduce_kernel<kOut><<<dim3(kTile * kTile / 4 / 256, static_cast<unsigned>(tail)), 256, 0, stream>>>(
        static_cast<const float*>(scratch), p, M, N, TM, TN, base, split);
    if (int status = check_launch("leaf products (tail reduction)")) return status;
  }
  if (layout.thin || (layout.strip && !persistent)) {
    thin::thin_rows_kernel<kIn, kOut>
        <<<dim3(static_cast<unsigned>(ceil_div(nb, thin::kCols)), static_cast<unsigned>(rank)), kGemmThreads, 0,
           stream>>>(A, B, p, M, N, K, static_cast<int>(tiles_m * kTile));
    if (int status = check_launch("leaf products (thin tile row)")) return status;
  }
  return FASTMM_OK;
}

}  // namespace fastmm

using namespace fastmm;

namespace fastmm {

// Kernel choice for one (operand, products) element-type pair.
template <int kIn, int kOut>
int launch_leaf_products(const void* a, const void* b, void* p, int64_t rank, int64_t mb, int64_t kb,
                         int64_t nb, void* scratch, int64_t scratch_bytes, hipStream_t s) {
  if (fast_leaf_gemm_applies(a, b, p, kb, nb, kOut) && mfma16_leaf_gemm_applies(mb, kb, nb)) {
    return launch_mfma16<kIn, kOut>(a, b, p, rank, mb, kb, nb, scratch, scratch_bytes, s);
  }
  if (fast_leaf_gemm_applies(a, b, p, kb, nb, kOut)) {
    return launch_tiles(fast::leaf_gemm_kernel<kIn, kOut>, fast::LDS_BYTES, a, b, p, rank, mb, kb, nb, s);
  }
  const bool aligned = kb % 8 == 0 && aligned_to(a, 16) && aligned_to(b, 16);
  if (slab_layout(kb)) {
    if (aligned) {
      return launch_tiles(generic::leaf_gemm_kernel<true, kIn, kOut, true>, generic::LDS_BYTES, a, b, p, rank,
                          mb, kb, nb, s);
    }
    return launch_tiles(generic::leaf_gemm_kernel<false, kIn, kOut, true>, generic::LDS_BYTES, a, b, p, rank,
                        mb, kb, nb, s);
  }
  if (aligned) {
    return launch_tiles(generic::leaf_gemm_kernel<true, kIn, kOut, false>, generic::LDS_BYTES, a, b, p, rank,
                        mb, kb, nb, s);
  }
  return launch_tiles(generic::leaf_gemm_kernel<false, kIn, kOut, false>, generic::LDS_BYTES, a, b, p, rank,
                      mb, kb, nb, s);
}

}  // namespace fastmm

namespace fastmm {

// Argument checks shared by both leaf-product entry points; FASTMM_OK or the error.
int check_leaf_arguments(int rank, int operand_dtype, const void* a, const void* b, const void* p,
                         int products_dtype, int64_t mb, int64_t kb, int64_t nb) {
  if (a == nullptr || b == nullptr || p == nullptr) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: null pointer");
  }
  if (rank < 1 || mb < 1 || kb < 1 || nb < 1) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: dimensions must be positive");
  }
  if (operand_dtype != kFP16 && operand_dtype != kBF16) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: operands must be fp16 or bf16");
  }
  if (products_dtype != operand_dtype && products_dtype != kFP32) {
    return fail(FASTMM_ERROR_ARGUMENT,
                "leaf products: products must be fp32 or the operands' type (%d), got %d",
                operand_dtype, products_dtype);
  }
  if (mb * kb > INT32_MAX || nb * kb > INT32_MAX || mb * nb > INT32_MAX) {
    return fail(FASTMM_ERROR_UNSUPPORTED, "leaf products: plane larger than 2^31 elements");
  }
  return FASTMM_OK;
}

// Element-type dispatch of checked arguments.
int run_leaf_products(int rank, int operand_dtype, const void* a, const void* b, void* p, int products_dtype,
                      int64_t mb, int64_t kb, int64_t nb, void* w, int64_t wb, hipStream_t s) {
  if (operand_dtype == kBF16) {
    if (products_dtype == kFP32) return launch_leaf_products<kBF16, kFP32>(a, b, p, rank, mb, kb, nb, w, wb, s);
    return launch_leaf_products<kBF16, kBF16>(a, b, p, rank, mb, kb, nb, w, wb, s);
  }
  if (products_dtype == kFP32) return launch_leaf_products<kFP16, kFP32>(a, b, p, rank, mb, kb, nb, w, wb, s);
  return launch_leaf_products<kFP16, kFP16>(a, b, p, rank, mb, kb, nb, w, wb, s);
}

// Split-K scratch bytes the 16x16x32 path plans for these arguments (0: no
// split tail), assuming 16-byte aligned buffers; the launcher re-checks the
// real pointers and runs the tail as whole tiles when they do not qualify.
int64_t planned_scratch_bytes(int rank, int products_dtype, int64_t mb, int64_t kb, int64_t nb) {
  const int64_t out_align = products_dtype == kFP32 ? 4 : 8;
  if (kb % fast::BK != 0 || kb < 3 * fast::BK || nb % out_align != 0 || !mfma16_leaf_gemm_applies(mb, kb, nb)) {
    return 0;
  }
  return tail_scratch_bytes(leaf_plan(rank, mb, kb, nb).split);
}

// ------------------------------------------------ allocation-free variant
//
// fastmm_leaf_products_noalloc keeps the split-K tail's fp32 parts in this
// file-scope device array instead of caller memory. Its size is the most the
// tail planner asks for on a 256-CU MI355X: at most 3/4 of the CUs' worth of
// parts (192), each one 256 x 256 fp32 tile. Every process that loads the
// library holds one copy per GPU it runs on until it exits. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// symbol): it uses the device address hipGetSymbolAddress returns, looked up
// once per device on that device's first call.
constexpr int64_t kStaticScratchBytes = int64_t{192} * kTile * kTile * static_cast<int64_t>(sizeof(float));
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_address[kMaxDevices];  // zero-initialized
std::mutex scratch_lookup;

// The current device's address of `scratch` (looked up on first use).
int static_scratch(void** address) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
    (void)hipGetLastError();
    return fail(FASTMM_ERROR_LAUNCH, "leaf products (no-alloc): no usable current device");
  }
  void* known = scratch_address[device].load(std::memory_order_acquire);
  if (known == nullptr) {
    std::lock_guard<std::mutex> guard(scratch_lookup);
    known = scratch_address[device].load(std::memory_order_acquire);
    if (known == nullptr) {
      const hipError_t status = hipGetSymbolAddress(&known, HIP_SYMBOL(scratch));
      if (status != hipSuccess || known == nullptr) {
        (void)hipGetLastError();
        return fail(FASTMM_ERROR_LAUNCH, "leaf products (no-alloc): scratch address on device %d: %s", device,
                    hipGetErrorString(status));
      }
      scratch_address[device].store(known, std::memory_order_release);
    }
  }
  *address = known;
  return FASTMM_OK;
}

}  // namespace fastmm

extern "C" int fastmm_leaf_products(int rank, int operand_dtype, const void* left_transformed,
                                    const void* right_transformed, void* products,
                                    int products_dtype, int64_t block_rows, int64_t block_inner,
                                    int64_t block_columns, void* scratch, int64_t scratch_bytes,
                                    void* stream) {
  clear_error();
  if (scratch_bytes < 0 || (scratch == nullptr && scratch_bytes != 0)) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: scratch of %lld bytes at null",
                static_cast<long long>(scratch_bytes));
  }
  if (int status = check_leaf_arguments(rank, operand_dtype, left_transformed, right_transformed, products,
                                        products_dtype, block_rows, block_inner, block_columns)) {
    return status;
  }
  return run_leaf_products(rank, operand_dtype, left_transformed, right_transformed, products, products_dtype,
                           block_rows, block_inner, block_columns, scratch, scratch_bytes,
                           static_cast<hipStream_t>(stream));
}

extern "C" int fastmm_leaf_products_noalloc(int rank, int operand_dtype, const void* left_transformed,
                                            const void* right_transformed, void* products, int products_dtype,
                                            int64_t block_rows, int64_t block_inner, int64_t block_columns,
                                            void* stream) {
  clear_error();
  if (int status = check_leaf_arguments(rank, operand_dtype, left_transformed, right_transformed, products,
                                        products_dtype, block_rows, block_inner, block_columns)) {
    return status;
  }
  const int64_t needed = planned_scratch_bytes(rank, products_dtype, block_rows, block_inner, block_columns);
  if (needed > kStaticScratchBytes) {
    return fail(FASTMM_ERROR_UNSUPPORTED,
                "leaf products (no-alloc): the split-K tail needs %lld bytes of scratch, above the library's "
                "static %lld; use fastmm_leaf_products with caller scratch",
                static_cast<long long>(needed), static_cast<long long>(kStaticScratchBytes));
  }
  void* address = nullptr;
  if (needed > 0) {
    if (int status = static_scratch(&address)) return status;
  }
  return run_leaf_products(rank, operand_dtype, left_transformed, right_transformed, products, products_dtype,
                           block_rows, block_inner, block_columns, address, needed,
                           static_cast<hipStream_t>(stream));
}

extern "C" int fastmm_leaf_scratch_bytes(int rank, int operand_dtype, int products_dtype, int64_t block_rows,
                                         int64_t block_inner, int64_t block_columns, int64_t* bytes) {
  clear_error();
  if (bytes == nullptr) return fail(FASTMM_ERROR_ARGUMENT, "leaf scratch bytes: null result pointer");
  *bytes = 0;
  if (rank < 1 || block_rows < 1 || block_inner < 1 || block_columns < 1) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf scratch bytes: dimensions must be positive");
  }
  if ((operand_dtype != kFP16 && operand_dtype != kBF16) ||
      (products_dtype != operand_dtype && products_dtype != kFP32)) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf scratch bytes: unsupported element types %d -> %d", operand_dtype,
                products_dtype);
  }
  // the split-K tail runs on the 16x16x32 path (16-byte aligned buffers assumed)
  *bytes = planned_scratch_bytes(rank, products_dtype, block_rows, block_inner, block_columns);
  return FASTMM_OK;
}
