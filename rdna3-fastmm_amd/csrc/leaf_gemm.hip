// Batched FP16 leaf products on CDNA4 MFMA (gfx950).
//
//   P[r] = A'[r] @ B'[r]^T,   A'[r]: [Mb, Kb], B'[r]: [Nb, Kb] (both K-contiguous)
//
// One workgroup (4 waves, 256 lanes) owns a BM x BN tile of one leaf. Each
// wave owns a (BM/2) x (BN/2) sub-tile as a grid of 32x32 accumulators fed by
// v_mfma_f32_32x32x16_f16 (fp32 accumulation). K advances in BK = 64 slices
// staged through LDS, double-buffered: the global loads of slice k+1 are in
// flight while the MFMAs of slice k run, and one barrier per slice separates
// the LDS write of one buffer from the reads of the other.
//
// LDS layout: a slice is BM (or BN) rows of 64 halves = 8 chunks of 16 bytes.
// Chunk c of row r lives at chunk position c ^ (r & 7), so the 16-byte reads
// of 8 consecutive rows at one k (the MFMA operand pattern) and the 16-byte
// writes of one row's 8 chunks both touch 8 distinct chunks = all 32 banks.
//
// MFMA operand convention: lane l supplies A[row l%32][k 8*(l/32) .. +7] and
// B'[row l%32][same k]; because A and B use one lane->k map the contraction
// is over all 16 k whatever order the hardware sums them in. The result
// layout is the documented 32x32 one: lane l, element e holds
// D[8*(e/4) + 4*(l/32) + e%4][l%32].
#include "abi_common.h"
#include "fastmm_device.h"

namespace fastmm {

constexpr int kGemmThreads = 256;
constexpr int kBK = 64;

template <int BM, int BN>
struct GemmShape {
  static constexpr int WM = BM / 2;  // wave tile rows (2 x 2 waves)
  static constexpr int WN = BN / 2;
  static constexpr int TM = WM / 32;  // 32x32 accumulators per wave
  static constexpr int TN = WN / 32;
  static constexpr int A_CHUNKS = BM * kBK / 8 / kGemmThreads;  // 16-byte loads per lane
  static constexpr int B_CHUNKS = BN * kBK / 8 / kGemmThreads;
  static constexpr int STAGE_HALVES = (BM + BN) * kBK;
  static constexpr int LDS_BYTES = 2 * STAGE_HALVES * 2;
};

__device__ __forceinline__ int swizzled(int row, int chunk) {
  return row * kBK + ((chunk ^ (row & 7)) << 3);
}

// Map the linear workgroup id to (leaf, tile_m, tile_n). Workgroups are
// dispatched round-robin over the 8 XCDs; renumber so each XCD works on a
// contiguous range of tiles (they share A rows / B rows in that XCD's L2),
// then walk tiles in column groups of `group` tile rows.
__device__ __forceinline__ void decode_tile(int wg, int total, int tiles_m, int tiles_n,
                                            int& leaf, int& tm, int& tn) {
  constexpr int kXcds = 8;
  int logical = wg;
  if (total % kXcds == 0) {
    const int per_xcd = total / kXcds;
    logical = (wg % kXcds) * per_xcd + wg / kXcds;
  }
  const int per_leaf = tiles_m * tiles_n;
  leaf = logical / per_leaf;
  int t = logical - leaf * per_leaf;
  constexpr int group = 4;
  const int group_span = group * tiles_n;
  const int g = t / group_span;
  const int first_m = g * group;
  const int rows_in_group = min(group, tiles_m - first_m);
  const int within = t - g * group_span;
  tm = first_m + within % rows_in_group;
  tn = within / rows_in_group;
}

template <int BM, int BN, bool kAligned, int kOut>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void leaf_gemm_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                      void* __restrict__ P, int Mb, int Nb, int Kb, int tiles_m, int tiles_n,
                      int total_tiles) {
  typedef GemmShape<BM, BN> G;
  extern __shared__ __attribute__((aligned(16))) half_t smem[];

  int leaf, tm, tn;
  decode_tile(blockIdx.x, total_tiles, tiles_m, tiles_n, leaf, tm, tn);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = tm * BM, n0 = tn * BN;
  const half_t* a_leaf = A + static_cast<int64_t>(leaf) * Mb * Kb;
  const half_t* b_leaf = B + static_cast<int64_t>(leaf) * Nb * Kb;

  uint4 a_regs[G::A_CHUNKS];
  uint4 b_regs[G::B_CHUNKS];

  auto load_rows = [&](const half_t* base, int row0, int rows, int k0, int chunks, uint4* regs) {
#pragma unroll
    for (int i = 0; i < chunks; ++i) {
      const int id = i * kGemmThreads + tid;
      const int row = id >> 3;
      const int k = k0 + ((id & 7) << 3);
      const int grow = row0 + row;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (grow < rows) {
        const half_t* p = base + static_cast<int64_t>(grow) * Kb + k;
        if constexpr (kAligned) {
          if (k < Kb) v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            h[e] = (k + e < Kb) ? __builtin_bit_cast(uint16_t, p[e]) : uint16_t{0};
          }
          __builtin_memcpy(&v, h, 16);
        }
      }
      regs[i] = v;
    }
  };
  auto global_load = [&](int k0) {
    load_rows(a_leaf, m0, Mb, k0, G::A_CHUNKS, a_regs);
    load_rows(b_leaf, n0, Nb, k0, G::B_CHUNKS, b_regs);
  };
  auto lds_store = [&](int buffer) {
    half_t* as = smem + buffer * G::STAGE_HALVES;
    half_t* bs = as + BM * kBK;
#pragma unroll
    for (int i = 0; i < G::A_CHUNKS; ++i) {
      const int id = i * kGemmThreads + tid;
      *reinterpret_cast<uint4*>(as + swizzled(id >> 3, id & 7)) = a_regs[i];
    }
#pragma unroll
    for (int i = 0; i < G::B_CHUNKS; ++i) {
      const int id = i * kGemmThreads + tid;
      *reinterpret_cast<uint4*>(bs + swizzled(id >> 3, id & 7)) = b_regs[i];
    }
  };

  float16v acc[G::TM][G::TN];
#pragma unroll
  for (int i = 0; i < G::TM; ++i)
#pragma unroll
    for (int j = 0; j < G::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int k_tiles = (Kb + kBK - 1) / kBK;
  global_load(0);
  lds_store(0);
  __syncthreads();

  const int lane_row = lane & 31;
  const int lane_chunk = lane >> 5;
  for (int kt = 0; kt < k_tiles; ++kt) {
    const int buffer = kt & 1;
    if (kt + 1 < k_tiles) global_load((kt + 1) * kBK);
    const half_t* as = smem + buffer * G::STAGE_HALVES;
    const half_t* bs = as + BM * kBK;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int chunk = 2 * ks + lane_chunk;
      half8 af[G::TM], bf[G::TN];
#pragma unroll
      for (int i = 0; i < G::TM; ++i) {
        const int row = wm * G::WM + i * 32 + lane_row;
        af[i] = *reinterpret_cast<const half8*>(as + swizzled(row, chunk));
      }
#pragma unroll
      for (int j = 0; j < G::TN; ++j) {
        const int row = wn * G::WN + j * 32 + lane_row;
        bf[j] = *reinterpret_cast<const half8*>(bs + swizzled(row, chunk));
      }
#pragma unroll
      for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < k_tiles) lds_store(buffer ^ 1);
    __syncthreads();
  }

  // Epilogue: lane l, element e of accumulator (i, j) is
  // row 8*(e/4) + 4*(l/32) + e%4, column l%32 of that 32x32 block.
  const int64_t leaf_offset = static_cast<int64_t>(leaf) * Mb * Nb;
#pragma unroll
  for (int i = 0; i < G::TM; ++i) {
#pragma unroll
    for (int j = 0; j < G::TN; ++j) {
      const int col = n0 + wn * G::WN + j * 32 + lane_row;
      if (col >= Nb) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * G::WM + i * 32 + 8 * (e >> 2) + 4 * lane_chunk + (e & 3);
        if (row < Mb) {
          const int64_t offset = leaf_offset + static_cast<int64_t>(row) * Nb + col;
          if constexpr (kOut == kFP32) {
            static_cast<float*>(P)[offset] = acc[i][j][e];
          } else {
            static_cast<uint16_t*>(P)[offset] = f32_to_fp16(acc[i][j][e]);
          }
        }
      }
    }
  }
}

template <int BM, int BN, bool kAligned, int kOut>
int launch_leaf_gemm(const void* a, const void* b, void* p, int64_t rank, int64_t mb, int64_t kb,
                     int64_t nb, hipStream_t stream) {
  typedef GemmShape<BM, BN> G;
  auto kernel = leaf_gemm_kernel<BM, BN, kAligned, kOut>;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            G::LDS_BYTES) != hipSuccess) {
      return fail(FASTMM_ERROR_LAUNCH, "leaf products: cannot reserve %d bytes of LDS",
                  G::LDS_BYTES);
    }
    configured = true;
  }
  const int64_t tiles_m = ceil_div(mb, BM);
  const int64_t tiles_n = ceil_div(nb, BN);
  const int64_t total = tiles_m * tiles_n * rank;
  if (total > INT32_MAX) return fail(FASTMM_ERROR_UNSUPPORTED, "leaf products: too many tiles");
  kernel<<<dim3(static_cast<unsigned>(total)), kGemmThreads, G::LDS_BYTES, stream>>>(
      static_cast<const half_t*>(a), static_cast<const half_t*>(b), p, static_cast<int>(mb),
      static_cast<int>(nb), static_cast<int>(kb), static_cast<int>(tiles_m),
      static_cast<int>(tiles_n), static_cast<int>(total));
  return check_launch("leaf products");
}

}  // namespace fastmm

using namespace fastmm;

extern "C" int fastmm_leaf_products(int rank, const void* left_transformed,
                                    const void* right_transformed, void* products,
                                    int products_dtype, int64_t block_rows, int64_t block_inner,
                                    int64_t block_columns, void* stream) {
  clear_error();
  if (left_transformed == nullptr || right_transformed == nullptr || products == nullptr) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: null pointer");
  }
  if (rank < 1 || block_rows < 1 || block_inner < 1 || block_columns < 1) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: dimensions must be positive");
  }
  if (products_dtype != kFP16 && products_dtype != kFP32) {
    return fail(FASTMM_ERROR_ARGUMENT, "leaf products: products must be fp16 or fp32");
  }
  if (block_rows * block_inner > INT32_MAX || block_columns * block_inner > INT32_MAX ||
      block_rows * block_columns > INT32_MAX) {
    return fail(FASTMM_ERROR_UNSUPPORTED, "leaf products: plane larger than 2^31 elements");
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool aligned = block_inner % 8 == 0 && aligned_to(left_transformed, 16) &&
                       aligned_to(right_transformed, 16);
  if (aligned) {
    if (products_dtype == kFP32) {
      return launch_leaf_gemm<256, 256, true, kFP32>(left_transformed, right_transformed, products,
                                                     rank, block_rows, block_inner,
                                                     block_columns, s);
    }
    return launch_leaf_gemm<256, 256, true, kFP16>(left_transformed, right_transformed, products,
                                                   rank, block_rows, block_inner, block_columns,
                                                   s);
  }
  if (products_dtype == kFP32) {
    return launch_leaf_gemm<256, 256, false, kFP32>(left_transformed, right_transformed, products,
                                                    rank, block_rows, block_inner, block_columns,
                                                    s);
  }
  return launch_leaf_gemm<256, 256, false, kFP16>(left_transformed, right_transformed, products,
                                                  rank, block_rows, block_inner, block_columns,
                                                  s);
}
