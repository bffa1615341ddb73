// Block transforms and output recombination for every scheme (gfx950).
//
// Transformed planes are written in the operand layout of fastmm_device.h
// (K-slab-major when Kb % 32 == 0, else row-major).
//
// All three kernels are HBM-bound elementwise passes over one block plane:
// a thread owns EPT consecutive plane elements (K-contiguous for the
// transforms, N-contiguous for the recombination), reads the s*s input
// blocks (or the R products) at that position with 8/16-byte vector loads,
// evaluates the scheme's straight-line program in fp32 registers, and writes
// every output with one vector store as soon as the program produces it.
// Positions past the matrix read as zero (the reference's masked loads with
// other=0.0). Programs come from csrc/generated/*.h.
#include <algorithm>

#include "abi_common.h"
#include "fastmm_device.h"
#include "generated/rank343_8x8x8.h"
#include "generated/rank48_4x4x4.h"
#include "generated/rank49_4x4x4.h"
#include "generated/rank7_2x2x2.h"

namespace fastmm {

constexpr int kThreads = 256;

// Elements per thread of the vector path: 8 (16-byte accesses) for the small
// rank-7 program; 4 for the 48/49-output programs and 2 for the 343-output
// programs, whose live fp32 values would otherwise spill.
template <class S>
constexpr int vector_width() { return S::kRank <= 8 ? 8 : S::kRank <= 64 ? 4 : 2; }

// The recombination reads R products per element: at R = 343, two fp16
// elements per thread fill the register file (two fp32 ones would spill, so
// fp32 products take one).
template <class S, int kProd>
constexpr int reconstruct_width() { return S::kRank <= 64 ? vector_width<S>() : kProd == kFP32 ? 1 : 2; }

// The 8x8-block schemes run in FP16 only (rank 343: FP16 operands, planes and
// output, as the reference's only precision pair); other element types are
// not instantiated for them.
template <class S>
constexpr bool fp16_only() { return S::kSize > 4; }

// Threads per workgroup of the transform and recombination passes.
template <class S>
constexpr int block_threads() { return kThreads; }

enum Side : int { kLeftSide = 0, kWeightSide = 1 };

// A' = left(x blocks) or B' = right(W^T blocks), read K-contiguous.
// Left:   input j = x block (j / s, j % s)      over x[src_rows, src_cols].
// Weight: input j = W^T block (j / s, j % s) = W block (j % s, j / s) over
//         W[src_rows = N, src_cols = K]; plane r of B' is [Nb, Kb].
// kPlane: element type of the transformed planes (kFP16 or kBF16, round to
// nearest even from the fp32 program value).
// kVector: src_cols == s * cols_b, cols_b % EPT == 0 and 2*EPT-aligned
// pointers, so every vector is wholly inside a row; otherwise EPT == 1.
// kSpan == 0: row-major output planes; a 1D grid walks them in storage order.
// kSpan == 32 or 64: K-slab-major output planes (cols_b % kSpan == 0); a 2D
// grid gives each wave RPW rows x kSpan columns, so a wave reads whole 64- or
// 128-byte line runs of every input row and writes RPW consecutive slab rows
// (RPW * 64 bytes) per slab and plane.
template <class S, int kSide, int kDType, int kPlane, int EPT, bool kVector, int kSpan>
__global__ __launch_bounds__(block_threads<S>()) void direct_transform_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int64_t src_rows,
    int64_t src_cols, int64_t rows_b, int64_t cols_b) {
  constexpr int s = S::kSize;
  const int64_t plane = rows_b * cols_b;
  int64_t row, col, at;
  if constexpr (kSpan == 0) {
    at = (static_cast<int64_t>(blockIdx.x) * block_threads<S>() + threadIdx.x) * EPT;
    if (at >= plane) return;
    row = at / cols_b;
    col = at - row * cols_b;
  } else {
    constexpr int CPR = kSpan / EPT, RPW = 64 / CPR;  // chunks per row, rows per wave
    static_assert(CPR * RPW == 64 && kSpan % kSlab == 0, "a wave covers whole slab rows");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    row = (static_cast<int64_t>(blockIdx.x) * (block_threads<S>() / 64) + wave) * RPW + lane / CPR;
    col = static_cast<int64_t>(blockIdx.y) * kSpan + (lane % CPR) * EPT;
    if (row >= rows_b) return;
    at = operand_offset<true>(row, col, rows_b, cols_b);
  }

  auto load = [&](int j) -> Vec<EPT> {
    const int block_row = kSide == kLeftSide ? j / s : j % s;
    const int block_col = kSide == kLeftSide ? j % s : j / s;
    const int64_t r = block_row * rows_b + row;
    const int64_t c = block_col * cols_b + col;
    // Branch-free: padding positions load a valid element (row 0, or the row's
    // last column) and select zero. A branch per input would put every load in
    // its own basic block, and the compiler would wait for each before issuing
    // the next (64 serialized round trips for an 8x8-block scheme).
    const bool row_inside = r < src_rows;
    const int64_t rr = row_inside ? r : 0;
    Vec<EPT> v;
    if constexpr (kVector) {
      v = load_vec<kDType, EPT>(src + rr * src_cols + c);
#pragma unroll
      for (int e = 0; e < EPT; ++e) v.v[e] = row_inside ? v.v[e] : 0.0f;
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const bool inside = row_inside && c + e < src_cols;
        const int64_t cc = c + e < src_cols ? c + e : src_cols - 1;
        const float value = to_f32<kDType>(src[rr * src_cols + cc]);
        v.v[e] = inside ? value : 0.0f;
      }
    }
    return v;
  };
  auto store = [&](int k, const Vec<EPT>& v) {
    store_vec<kPlane, EPT>(dst + k * plane + at, v);
  };
  if constexpr (kSide == kLeftSide) {
    S::template left<Vec<EPT>>(load, store);
  } else {
    S::template right<Vec<EPT>>(load, store);
  }
}

// B' from a row-major right[K, N] (the mm path): the blocks are N-contiguous
// in memory but B' planes are K-contiguous, so a 32x32 (k, n) tile of every
// input block is staged through LDS and read transposed. In the K-slab
// layout a tile's output is one contiguous 2 KB block per plane.
constexpr int kTransposeTile = 32;
static_assert(kTransposeTile == kSlab, "a transpose tile covers exactly one K slab");

// Tile width in n: 32 columns of every input block for s <= 4 (s*s*32*33 fp32
// = 67.6 KB of LDS at s = 4); 8 columns for s = 8, whose 64 input blocks
// would need 270 KB at 32.
template <class S>
constexpr int transpose_columns() { return S::kSize <= 4 ? 32 : 8; }

template <class S, int kDType, int kPlane, bool kSlabLayout>
__global__ __launch_bounds__(kThreads) void transposed_right_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int64_t inner,
    int64_t columns, int64_t kb, int64_t nb) {
  constexpr int s = S::kSize;
  constexpr int T = kTransposeTile;
  constexpr int TN = transpose_columns<S>();
  constexpr int EK = T * TN / kThreads;  // k values per thread in the program pass
  static_assert(EK >= 1 && T * TN % kThreads == 0, "the block covers the tile exactly");
  __shared__ float tile[s * s][T][TN + 1];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * TN;
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * T;
  const int tid = threadIdx.x;
  const int nn = tid % TN;
#pragma unroll
  for (int j = 0; j < s * s; ++j) {
    const int64_t block_k = j / s, block_n = j % s;
#pragma unroll
    for (int pass = 0; pass < T * TN / kThreads; ++pass) {
      const int kk = tid / TN + pass * (kThreads / TN);
      const int64_t k = k0 + kk, n = n0 + nn;
      const int64_t src_row = block_k * kb + k, src_col = block_n * nb + n;
      // branch-free (see direct_transform_kernel): padding loads element 0
      const bool inside = k < kb && n < nb && src_row < inner && src_col < columns;
      const float value = to_f32<kDType>(src[inside ? src_row * columns + src_col : 0]);
      tile[j][kk][nn] = inside ? value : 0.0f;
    }
  }
  __syncthreads();
  const int n_local = tid / (T / EK);
  const int k_local = (tid % (T / EK)) * EK;
  auto load = [&](int j) -> Vec<EK> {
    Vec<EK> v;
#pragma unroll
    for (int e = 0; e < EK; ++e) v.v[e] = tile[j][k_local + e][n_local];
    return v;
  };
  const int64_t n = n0 + n_local;
  const int64_t k = k0 + k_local;
  auto store = [&](int r, const Vec<EK>& v) {
    if (n >= nb) return;
    uint16_t* p = dst + static_cast<int64_t>(r) * nb * kb + operand_offset<kSlabLayout>(n, k, nb, kb);
#pragma unroll
    for (int e = 0; e < EK; ++e) {
      if (k + e < kb) p[e] = from_f32<kPlane>(v.v[e]);
    }
  };
  S::template right<Vec<EK>>(load, store);
}

// C = output(P planes) (+ bias), stored as kOut. One thread: EPT consecutive
// columns of one product-plane row, i.e. the same EPT columns of s output
// rows... of every output block at that position.
template <int kProd, int EPT>
__device__ __forceinline__ Vec<EPT> load_product(const void* products, int64_t offset) {
  if constexpr (kProd == kFP32) {
    const float* p = static_cast<const float*>(products) + offset;
    Vec<EPT> v;
    if constexpr (EPT % 4 == 0) {
#pragma unroll
      for (int e = 0; e < EPT; e += 4) {
        const float4 q = *reinterpret_cast<const float4*>(p + e);
        v.v[e] = q.x;
        v.v[e + 1] = q.y;
        v.v[e + 2] = q.z;
        v.v[e + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) v.v[e] = p[e];
    }
    return v;
  } else {
    return load_vec<kProd, EPT>(static_cast<const uint16_t*>(products) + offset);
  }
}

// The output is stored with streaming stores: it is written once, and kept out
// of the caches it leaves them to the next call's transform input (C4: that
// transform 0.113 ms after this kernel against 0.145 ms after plain stores).
// kStreamIn: the vector path's product loads stream too; the launcher sets it
// when the products exceed the Infinity Cache, which then cannot still hold
// the leaf GEMM's freshly written products (C4's 2.0 GB of products
// recombine in 0.441 ms streamed, 0.496 ms plain; 0.13-0.23 GB, which stay
// cached, recombine 3-10 % slower streamed).
template <class S, int kProd, int kOut, int EPT, bool kVector, bool kBias, bool kStreamIn = false>
__global__ __launch_bounds__(block_threads<S>()) void reconstruct_kernel(
    const void* __restrict__ products, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int64_t rows, int64_t cols, int64_t rows_b, int64_t cols_b) {
  constexpr int s = S::kSize;
  const int64_t plane = rows_b * cols_b;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * block_threads<S>() + threadIdx.x) * EPT;
  if (first >= plane) return;
  const int64_t row = first / cols_b;
  const int64_t col = first - row * cols_b;

  // Vector path with 16-bit products and R <= 64: every product (and bias)
  // load is issued before the program runs and kept as raw bits (two
  // registers per product at EPT = 4). Evaluated lazily, the late loads each
  // come right before their first use, so every one waits a full memory round
  // trip. Same arithmetic either way.
  if constexpr (kVector && kProd != kFP32 && S::kRank <= 64) {
    typedef typename Raw16<EPT>::type Raw;
    const uint16_t* base = static_cast<const uint16_t*>(products) + first;
    Raw raw[S::kRank];
#pragma unroll
    for (int r = 0; r < S::kRank; ++r) {
      const uint16_t* at = base + static_cast<int64_t>(r) * plane;
      if constexpr (kStreamIn) {
        raw[r] = load_raw16_stream<EPT>(at);
      } else {
        raw[r] = *reinterpret_cast<const Raw*>(at);
      }
    }
    Raw bias_raw[kBias ? s : 1];
    if constexpr (kBias) {
#pragma unroll
      for (int j = 0; j < s; ++j) bias_raw[j] = *reinterpret_cast<const Raw*>(bias + j * cols_b + col);
    }
    asm volatile("" ::: "memory");  // no load moves below this point
    auto load = [&](int r) -> Vec<EPT> { return raw_to_vec<kProd, EPT>(raw[r]); };
    auto store = [&](int c, Vec<EPT> v) {
      const int64_t out_row = (c / s) * rows_b + row;
      if (out_row >= rows) return;
      const int64_t out_col = (c % s) * cols_b + col;
      if constexpr (kBias) v = v + raw_to_vec<kOut, EPT>(bias_raw[c % s]);
      store_vec<kOut, EPT, true>(out + out_row * cols + out_col, v);
    };
    S::template output<Vec<EPT>>(load, store);
    return;
  }

  auto load = [&](int r) -> Vec<EPT> {
    return load_product<kProd, EPT>(products, static_cast<int64_t>(r) * plane + first);
  };
  auto store = [&](int c, Vec<EPT> v) {
    const int64_t out_row = (c / s) * rows_b + row;
    if (out_row >= rows) return;
    const int64_t out_col = (c % s) * cols_b + col;
    uint16_t* p = out + out_row * cols + out_col;
    if constexpr (kVector) {
      if constexpr (kBias) {
        const Vec<EPT> b = load_vec<kOut, EPT>(bias + out_col);
        v = v + b;
      }
      store_vec<kOut, EPT, true>(p, v);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if (out_col + e < cols) {
          float value = v.v[e];
          if constexpr (kBias) value = value + to_f32<kOut>(bias[out_col + e]);
          p[e] = from_f32<kOut>(value);
        }
      }
    }
  };
  S::template output<Vec<EPT>>(load, store);
}

// ------------------------------------------- dense recombination (8x8 blocks)

// The 8x8-block scheme's recombination as one dense contraction, the form the
// reference runs (generated/rank343_8x8x8.py output_transform_mfma_kernel,
// runtime.py:938-962): C block c = sum over r of M[c][r] * P[r], with fp16
// products and coefficients (-1, 0, 1) multiplied on FP16 MFMA
// (v_mfma_f32_16x16x32_f16), summed in fp32 and rounded once to the fp16
// output. Every term is exact in fp32; only the fp32 summation order is the
// hardware's. Rank-padded K runs over ceil(R / 32) steps of 32 products.
//
// One wave owns 64 plane positions per tile and all 64 outputs (4 x 4 MFMA
// tiles of 16 positions x 16 outputs). Per K step it loads 32 products x 64
// positions (a lane: 4 products x 8 positions, 16-byte loads), writes them
// transposed into its own LDS stage (position-major, 32 products per row) and
// reads the MFMA fragments back as 16-byte rows. The coefficient matrix sits
// in LDS as fp16 for the whole kernel. Loads run kDepth K steps ahead.
namespace dense {

constexpr int kWaves = 4;
constexpr int kPositions = 64;              // plane positions per wave and tile
constexpr int kStep = 32;                   // products per MFMA K step
constexpr int kStageRow = kStep * 2 + 16;   // bytes per staged position; the pad keeps the
                                            // 16 rows a fragment read touches on distinct banks
constexpr int kDepth = 6;                   // K steps of loads in flight per wave

template <class S>
constexpr int steps() { return (S::kRank + kStep - 1) / kStep; }
// Bytes per output row of the staged matrix (padded like the stage rows).
template <class S>
constexpr int matrix_row() { return steps<S>() * kStep * 2 + 16; }
template <class S>
constexpr int lds_bytes() { return S::kSize * S::kSize * matrix_row<S>() + kWaves * kPositions * kStageRow; }

__device__ __forceinline__ uint32_t component(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Requires cols == s * cols_b, cols_b % 8 == 0 (so plane % 8 == 0 and every
// group of 8 positions lies in one plane row), 16-byte aligned products and an
// 8-byte aligned output; the launcher checks all four.
template <class S>
__global__ __launch_bounds__(kWaves * 64) void dense_reconstruct_kernel(
    const uint16_t* __restrict__ products, uint16_t* __restrict__ out, int64_t rows, int64_t cols,
    int64_t rows_b, int64_t cols_b, int64_t tiles) {
  constexpr int R = S::kRank, s = S::kSize, KS = steps<S>(), KP = KS * kStep;
  constexpr int MROW = matrix_row<S>();
  static_assert(s * s == 64, "four 16-output MFMA column blocks");
  __shared__ __attribute__((aligned(16))) unsigned char lds[lds_bytes<S>()];
  // M[c][r] as fp16 at c * MROW + 2 r, zero for r >= R
  for (int i = threadIdx.x; i < s * s * KP; i += kWaves * 64) {
    const int c = i / KP, r = i - c * KP;
    const float m = r < R ? static_cast<float>(S::kOutputMatrix[c][r]) : 0.0f;
    *reinterpret_cast<half_t*>(lds + c * MROW + 2 * r) = static_cast<half_t>(m);
  }
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  unsigned char* stage = lds + s * s * MROW + wave * kPositions * kStageRow;
  const int64_t plane = rows_b * cols_b;
  const int group = lane >> 3;               // loads products 4 group + j of each K step
  const int span = lane & 7;                 // for tile positions 8 span .. 8 span + 7
  const int fr = lane & 15, fk = lane >> 4;  // fragment row, 8-wide K chunk

  for (int64_t tile = static_cast<int64_t>(blockIdx.x) * kWaves + wave; tile < tiles;
       tile += static_cast<int64_t>(gridDim.x) * kWaves) {
    const int64_t p0 = tile * kPositions;
    const int64_t pos = p0 + 8 * span;
    // Positions past the plane (plane % 8 == 0: whole groups) read position 0:
    // a position's outputs depend on its own products only, and these are
    // never stored. Products past R read product R - 1 and are zeroed (their
    // coefficients are zero, but an Inf or NaN there would still poison the
    // sum). Branch-free, so the loads pipeline.
    const uint16_t* lane_products = products + (pos < plane ? pos : 0);
    uint4 v[KS][4];
    auto fetch = [&](int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = ks * kStep + 4 * group + j;
        v[ks][j] = *reinterpret_cast<const uint4*>(lane_products + static_cast<int64_t>(r < R ? r : R - 1) * plane);
      }
    };
#pragma unroll
    for (int ks = 0; ks < kDepth && ks < KS; ++ks) fetch(ks);
    float4v acc[4][4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) acc[pb][cb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + kDepth < KS) fetch(ks + kDepth);
      uint32_t d[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool keep = (ks + 1) * kStep <= R || ks * kStep + 4 * group + j < R;
#pragma unroll
        for (int i = 0; i < 4; ++i) d[j][i] = keep ? component(v[ks][j], i) : 0u;
      }
      // position 8 span + q: products 4 group .. 4 group + 3 as one 8-byte row piece
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = q >> 1;
        const uint32_t lo = (q & 1) ? (d[0][i] >> 16) | (d[1][i] & 0xffff0000u) : (d[0][i] & 0xffffu) | (d[1][i] << 16);
        const uint32_t hi = (q & 1) ? (d[2][i] >> 16) | (d[3][i] & 0xffff0000u) : (d[2][i] & 0xffffu) | (d[3][i] << 16);
        *reinterpret_cast<uint2*>(stage + (8 * span + q) * kStageRow + 8 * group) = make_uint2(lo, hi);
      }
      // A = P^T fragments (row: position 16 pb + fr), B = M^T fragments (column:
      // output 16 cb + fr); lane l holds K values 8 fk .. 8 fk + 7 of its row.
      uint4 a[4], b[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
        a[pb] = *reinterpret_cast<const uint4*>(stage + (16 * pb + fr) * kStageRow + 16 * fk);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        b[cb] = *reinterpret_cast<const uint4*>(lds + (16 * cb + fr) * MROW + 2 * (ks * kStep + 8 * fk));
#pragma unroll
      for (int pb = 0; pb < 4; ++pb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          acc[pb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(half8, a[pb]), __builtin_bit_cast(half8, b[cb]), acc[pb][cb], 0, 0, 0);
    }
    // Element e of acc[pb][cb] in lane l: output block 16 cb + fr at plane
    // position p0 + 16 pb + 4 fk + e (four consecutive columns of one row).
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      const int64_t p = p0 + 16 * pb + 4 * fk;
      if (p >= plane) continue;
      const int64_t row = p / cols_b, col = p - row * cols_b;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int c = 16 * cb + fr;
        const int64_t out_row = (c / s) * rows_b + row;
        if (out_row >= rows) continue;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = f32_to_fp16(acc[pb][cb][e]);
        store16<4>(out + out_row * cols + (c % s) * cols_b + col, h);
      }
    }
  }
}

}  // namespace dense

// ------------------------------------------------------------- launchers

template <class S>
int launch_direct(int side, int dtype, int plane_dtype, const void* src, void* dst, int64_t src_rows,
                  int64_t src_cols, hipStream_t stream) {
  constexpr int s = S::kSize;
  constexpr int W = vector_width<S>();
  constexpr int B = block_threads<S>();
  const int64_t rows_b = ceil_div(src_rows, s);
  const int64_t cols_b = ceil_div(src_cols, s);
  const bool vector = src_cols % (s * W) == 0 && aligned_to(src, 2 * W) && aligned_to(dst, 2 * W);
  const int64_t plane = rows_b * cols_b;
  const uint16_t* in = static_cast<const uint16_t*>(src);
  uint16_t* out = static_cast<uint16_t*>(dst);
  const int span = !slab_layout(cols_b) ? 0 : cols_b % 64 == 0 ? 64 : 32;
  if (span != 0 && cols_b / span > 65535) {
    return fail(FASTMM_ERROR_UNSUPPORTED, "transform: inner dimension too large for the K-span grid");
  }
  // 1D grid over the plane (row-major) or 2D grid of (4 waves x RPW rows) x kSpan columns
  auto grid_for = [&](int ept, int kspan) {
    if (kspan == 0) return dim3(static_cast<unsigned>(ceil_div(plane, static_cast<int64_t>(B) * ept)));
    const int64_t rows_per_block = static_cast<int64_t>(B / 64) * (64 / (kspan / ept));
    return dim3(static_cast<unsigned>(ceil_div(rows_b, rows_per_block)), static_cast<unsigned>(cols_b / kspan));
  };
#define FASTMM_DIRECT_LAYOUT(SIDE, DT, PL, SPAN)                                              \
  do {                                                                                        \
    if (vector)                                                                               \
      direct_transform_kernel<S, SIDE, DT, PL, W, true, SPAN><<<grid_for(W, SPAN), B, 0,        \
                                                                 stream>>>(in, out, src_rows,  \
                                                                           src_cols, rows_b,   \
                                                                           cols_b);            \
    else                                                                                      \
      direct_transform_kernel<S, SIDE, DT, PL, 1, false, SPAN><<<grid_for(1, SPAN), B,          \
                                                                  0, stream>>>(in, out,        \
                                                                               src_rows,       \
                                                                               src_cols,       \
                                                                               rows_b, cols_b); \
  } while (0)
#define FASTMM_DIRECT_PLANE(SIDE, DT, PL)                                                     \
  do {                                                                                        \
    if (span == 64) FASTMM_DIRECT_LAYOUT(SIDE, DT, PL, 64);                                   \
    else if (span == 32) FASTMM_DIRECT_LAYOUT(SIDE, DT, PL, 32);                              \
    else FASTMM_DIRECT_LAYOUT(SIDE, DT, PL, 0);                                               \
  } while (0)
#define FASTMM_DIRECT(SIDE, DT)                                                               \
  do {                                                                                        \
    if (plane_dtype == kBF16) FASTMM_DIRECT_PLANE(SIDE, DT, kBF16);                           \
    else FASTMM_DIRECT_PLANE(SIDE, DT, kFP16);                                                \
  } while (0)
  if constexpr (fp16_only<S>()) {
    if (dtype != kFP16 || plane_dtype != kFP16) {
      return fail(FASTMM_ERROR_UNSUPPORTED, "transform: the %dx%d-block scheme takes fp16 input and planes",
                  s, s);
    }
    if (side == kLeftSide) FASTMM_DIRECT_PLANE(kLeftSide, kFP16, kFP16);
    else FASTMM_DIRECT_PLANE(kWeightSide, kFP16, kFP16);
  } else if (side == kLeftSide) {
    if (dtype == kBF16) FASTMM_DIRECT(kLeftSide, kBF16);
    else FASTMM_DIRECT(kLeftSide, kFP16);
  } else {
    if (dtype == kBF16) FASTMM_DIRECT(kWeightSide, kBF16);
    else FASTMM_DIRECT(kWeightSide, kFP16);
  }
#undef FASTMM_DIRECT
#undef FASTMM_DIRECT_PLANE
#undef FASTMM_DIRECT_LAYOUT
  return check_launch(side == kLeftSide ? "left transform" : "weight transform");
}

template <class S>
int launch_transposed(int dtype, int plane_dtype, const void* src, void* dst, int64_t inner,
                      int64_t columns, hipStream_t stream) {
  constexpr int s = S::kSize;
  const int64_t kb = ceil_div(inner, s);
  const int64_t nb = ceil_div(columns, s);
  const dim3 grid(static_cast<unsigned>(ceil_div(nb, static_cast<int64_t>(transpose_columns<S>()))),
                  static_cast<unsigned>(ceil_div(kb, kTransposeTile)));
  const uint16_t* in = static_cast<const uint16_t*>(src);
  uint16_t* out = static_cast<uint16_t*>(dst);
  const bool slab = slab_layout(kb);
#define FASTMM_TRANSPOSED(DT, PL)                                                                       \
  do {                                                                                                  \
    if (slab) transposed_right_kernel<S, DT, PL, true><<<grid, kThreads, 0, stream>>>(in, out, inner,   \
                                                                                       columns, kb, nb); \
    else transposed_right_kernel<S, DT, PL, false><<<grid, kThreads, 0, stream>>>(in, out, inner,       \
                                                                                   columns, kb, nb);     \
  } while (0)
  if constexpr (fp16_only<S>()) {
    if (dtype != kFP16 || plane_dtype != kFP16) {
      return fail(FASTMM_ERROR_UNSUPPORTED, "right transform: the %dx%d-block scheme takes fp16 input and planes",
                  s, s);
    }
    FASTMM_TRANSPOSED(kFP16, kFP16);
  } else if (dtype == kBF16) {
    if (plane_dtype == kBF16) FASTMM_TRANSPOSED(kBF16, kBF16);
    else FASTMM_TRANSPOSED(kBF16, kFP16);
  } else {
    if (plane_dtype == kBF16) FASTMM_TRANSPOSED(kFP16, kBF16);
    else FASTMM_TRANSPOSED(kFP16, kFP16);
  }
#undef FASTMM_TRANSPOSED
  return check_launch("right transform");
}

// Products larger than this stream past the caches in the recombination: the
// MI355X Infinity Cache holds 256 MiB.
constexpr int64_t kStreamProductBytes = int64_t{256} << 20;

template <class S, int kProd, int kOut, bool kBias>
void launch_reconstruct_typed(bool vector, dim3 grid, hipStream_t stream, const void* products,
                              const uint16_t* bias, uint16_t* out, int64_t rows, int64_t cols,
                              int64_t rows_b, int64_t cols_b) {
  constexpr int W = reconstruct_width<S, kProd>();
  if (vector) {
    constexpr bool kCanStream = kProd != kFP32 && S::kRank <= 64;  // the raw-bits load path
    const int64_t product_bytes = static_cast<int64_t>(S::kRank) * rows_b * cols_b * 2;
    if (kCanStream && product_bytes > kStreamProductBytes) {
      reconstruct_kernel<S, kProd, kOut, W, true, kBias, kCanStream>
          <<<grid, block_threads<S>(), 0, stream>>>(products, bias, out, rows, cols, rows_b, cols_b);
    } else {
      reconstruct_kernel<S, kProd, kOut, W, true, kBias>
          <<<grid, block_threads<S>(), 0, stream>>>(products, bias, out, rows, cols, rows_b, cols_b);
    }
  } else {
    reconstruct_kernel<S, kProd, kOut, 1, false, kBias>
        <<<grid, block_threads<S>(), 0, stream>>>(products, bias, out, rows, cols, rows_b, cols_b);
  }
}

template <class S>
int launch_reconstruct(int products_dtype, const void* products, const void* bias, int dtype,
                       void* output, int64_t rows, int64_t cols, hipStream_t stream) {
  constexpr int s = S::kSize;
  const int W = products_dtype == kFP32 ? reconstruct_width<S, kFP32>() : reconstruct_width<S, kFP16>();
  const int64_t rows_b = ceil_div(rows, s);
  const int64_t cols_b = ceil_div(cols, s);
  const int product_bytes = products_dtype == kFP32 ? 4 : 2;
  const bool vector = cols % (s * W) == 0 && aligned_to(products, product_bytes * W) &&
                      aligned_to(output, 2 * W) && (bias == nullptr || aligned_to(bias, 2 * W));
  const int64_t plane = rows_b * cols_b;
  const int64_t per_block = static_cast<int64_t>(block_threads<S>()) * (vector ? W : 1);
  const dim3 grid(static_cast<unsigned>(ceil_div(plane, per_block)));
  const uint16_t* b = static_cast<const uint16_t*>(bias);
  uint16_t* out = static_cast<uint16_t*>(output);
#define FASTMM_RECON(PROD, OUT)                                                                 \
  do {                                                                                          \
    if (b)                                                                                      \
      launch_reconstruct_typed<S, PROD, OUT, true>(vector, grid, stream, products, b, out,      \
                                                   rows, cols, rows_b, cols_b);                 \
    else                                                                                        \
      launch_reconstruct_typed<S, PROD, OUT, false>(vector, grid, stream, products, b, out,     \
                                                    rows, cols, rows_b, cols_b);                \
  } while (0)
  if constexpr (fp16_only<S>()) {
    if (dtype != kFP16 || products_dtype == kBF16) {
      return fail(FASTMM_ERROR_UNSUPPORTED,
                  "reconstruct: the %dx%d-block scheme takes fp16 or fp32 products and an fp16 output", s, s);
    }
    // fp16 products, no bias, whole 8-column position groups: the dense MFMA
    // form (the reference's); otherwise the output circuit below.
    if (products_dtype == kFP16 && b == nullptr && cols == s * cols_b && cols_b % 8 == 0 &&
        aligned_to(products, 16) && aligned_to(output, 8)) {
      const int64_t tiles = ceil_div(plane, dense::kPositions);
      const int cus = compute_units();  // two 4-wave workgroups fit a CU's LDS
      const int64_t resident = 2 * static_cast<int64_t>(cus > 0 ? cus : 256);
      const dim3 dense_grid(static_cast<unsigned>(std::min(ceil_div(tiles, dense::kWaves), resident)));
      dense::dense_reconstruct_kernel<S><<<dense_grid, dense::kWaves * 64, 0, stream>>>(
          static_cast<const uint16_t*>(products), out, rows, cols, rows_b, cols_b, tiles);
      return check_launch("reconstruct");
    }
    if (products_dtype == kFP32) FASTMM_RECON(kFP32, kFP16);
    else FASTMM_RECON(kFP16, kFP16);
  } else if (products_dtype == kFP32) {
    if (dtype == kBF16) FASTMM_RECON(kFP32, kBF16);
    else FASTMM_RECON(kFP32, kFP16);
  } else if (products_dtype == kBF16) {
    if (dtype == kBF16) FASTMM_RECON(kBF16, kBF16);
    else FASTMM_RECON(kBF16, kFP16);
  } else {
    if (dtype == kBF16) FASTMM_RECON(kFP16, kBF16);
    else FASTMM_RECON(kFP16, kFP16);
  }
#undef FASTMM_RECON
  return check_launch("reconstruct");
}

// Calls f.template operator()<Scheme>() for the scheme id, or fails.
template <class F>
int with_scheme(int scheme, F&& f) {
  switch (scheme) {
    case FASTMM_SCHEME_RANK7: return f.template operator()<SchemeRank7>();
    case FASTMM_SCHEME_RANK48: return f.template operator()<SchemeRank48>();
    case FASTMM_SCHEME_RANK49: return f.template operator()<SchemeRank49>();
    case FASTMM_SCHEME_RANK343: return f.template operator()<SchemeRank343>();
    default: return fail(FASTMM_ERROR_ARGUMENT, "unknown scheme id %d", scheme);
  }
}

int check_plane_dtype(const char* name, int plane_dtype) {
  if (plane_dtype != kFP16 && plane_dtype != kBF16) {
    return fail(FASTMM_ERROR_ARGUMENT, "%s: planes must be fp16 or bf16, got %d", name, plane_dtype);
  }
  return FASTMM_OK;
}

int check_io(const char* name, int dtype, const void* a, const void* b, int64_t rows,
             int64_t cols) {
  if (dtype != kBF16 && dtype != kFP16) {
    return fail(FASTMM_ERROR_ARGUMENT, "%s: dtype must be bf16 or fp16, got %d", name, dtype);
  }
  if (a == nullptr || b == nullptr) return fail(FASTMM_ERROR_ARGUMENT, "%s: null pointer", name);
  if (rows < 1 || cols < 1) {
    return fail(FASTMM_ERROR_ARGUMENT, "%s: dimensions must be positive", name);
  }
  if (rows > (int64_t{1} << 31) || cols > (int64_t{1} << 31)) {
    return fail(FASTMM_ERROR_UNSUPPORTED, "%s: dimension too large", name);
  }
  return FASTMM_OK;
}

}  // namespace fastmm

using namespace fastmm;

extern "C" int fastmm_scheme_info(int scheme, int* size, int* rank) {
  clear_error();
  return with_scheme(scheme, [&]<class S>() {
    if (size) *size = S::kSize;
    if (rank) *rank = S::kRank;
    return FASTMM_OK;
  });
}

extern "C" const char* fastmm_scheme_sha256(int scheme) {
  switch (scheme) {
    case FASTMM_SCHEME_RANK7: return SchemeRank7::kCertificateSha256;
    case FASTMM_SCHEME_RANK48: return SchemeRank48::kCertificateSha256;
    case FASTMM_SCHEME_RANK49: return SchemeRank49::kCertificateSha256;
    case FASTMM_SCHEME_RANK343: return SchemeRank343::kCertificateSha256;
    default: return nullptr;
  }
}

extern "C" int fastmm_left_transform(int scheme, int dtype, int plane_dtype, const void* input,
                                     void* left_transformed, int64_t rows, int64_t inner,
                                     void* stream) {
  clear_error();
  if (int status = check_io("left transform", dtype, input, left_transformed, rows, inner)) {
    return status;
  }
  if (int status = check_plane_dtype("left transform", plane_dtype)) return status;
  return with_scheme(scheme, [&]<class S>() {
    return launch_direct<S>(kLeftSide, dtype, plane_dtype, input, left_transformed, rows, inner,
                            static_cast<hipStream_t>(stream));
  });
}

extern "C" int fastmm_weight_transform(int scheme, int dtype, int plane_dtype, const void* weight,
                                       void* right_transformed, int64_t columns, int64_t inner,
                                       void* stream) {
  clear_error();
  if (int status =
          check_io("weight transform", dtype, weight, right_transformed, columns, inner)) {
    return status;
  }
  if (int status = check_plane_dtype("weight transform", plane_dtype)) return status;
  return with_scheme(scheme, [&]<class S>() {
    return launch_direct<S>(kWeightSide, dtype, plane_dtype, weight, right_transformed, columns,
                            inner, static_cast<hipStream_t>(stream));
  });
}

extern "C" int fastmm_right_transform(int scheme, int dtype, int plane_dtype, const void* right,
                                      void* right_transformed, int64_t inner, int64_t columns,
                                      void* stream) {
  clear_error();
  if (int status = check_io("right transform", dtype, right, right_transformed, inner, columns)) {
    return status;
  }
  if (int status = check_plane_dtype("right transform", plane_dtype)) return status;
  return with_scheme(scheme, [&]<class S>() {
    return launch_transposed<S>(dtype, plane_dtype, right, right_transformed, inner, columns,
                                static_cast<hipStream_t>(stream));
  });
}

extern "C" int fastmm_reconstruct(int scheme, int products_dtype, const void* products,
                                  const void* bias, int dtype, void* output, int64_t rows,
                                  int64_t columns, void* stream) {
  clear_error();
  if (int status = check_io("reconstruct", dtype, products, output, rows, columns)) {
    return status;
  }
  if (products_dtype != kFP16 && products_dtype != kBF16 && products_dtype != kFP32) {
    return fail(FASTMM_ERROR_ARGUMENT, "reconstruct: products must be fp16, bf16 or fp32");
  }
  return with_scheme(scheme, [&]<class S>() {
    return launch_reconstruct<S>(products_dtype, products, bias, dtype, output, rows, columns,
                                 static_cast<hipStream_t>(stream));
  });
}
