// Device-side building blocks shared by the fast-matmul kernels (gfx950).
#ifndef FASTMM_DEVICE_H
#define FASTMM_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fastmm {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

// Element codes shared with the C ABI (include/fastmm_amd.h).
enum DType : int { kBF16 = 0, kFP16 = 1, kFP32 = 2 };

// ---------------------------------------------------------- operand layout

// Transformed operand planes (A' is [Mb, Kb], B' is [Nb, Kb]) are stored
// K-slab-major when Kb is a multiple of 32: element (row, k) of a plane with
// `rows` rows sits at ((k / 32) * rows + row) * 32 + k % 32, so the 32-wide K
// slice of any run of rows is one contiguous block (a leaf-GEMM tile's slice
// is 16 KB of consecutive bytes instead of 64-byte pieces of 256 rows). Other
// Kb keep row-major planes.
constexpr int kSlab = 32;

__host__ __device__ __forceinline__ bool slab_layout(int64_t inner) { return inner % kSlab == 0; }

template <bool kSlabLayout>
__host__ __device__ __forceinline__ int64_t operand_offset(int64_t row, int64_t k, int64_t rows,
                                                           int64_t inner) {
  if constexpr (kSlabLayout) return ((k / kSlab) * rows + row) * kSlab + k % kSlab;
  else return row * inner + k;
}

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN. Both results
// are computed and one selected (no branch: vectorized callers keep every
// lane on one path).
__device__ __forceinline__ uint16_t f32_to_bf16(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t quiet = (bits >> 16) | 0x40u;
  const uint32_t rounded = (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
  return static_cast<uint16_t>((bits & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

__device__ __forceinline__ float fp16_to_f32(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(half_t, bits));
}

// fp32 -> fp16 with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint16_t f32_to_fp16(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<half_t>(value));
}

template <int kDType>
__device__ __forceinline__ float to_f32(uint16_t bits) {
  if constexpr (kDType == kBF16) return bf16_to_f32(bits);
  else return fp16_to_f32(bits);
}

template <int kDType>
__device__ __forceinline__ uint16_t from_f32(float value) {
  if constexpr (kDType == kBF16) return f32_to_bf16(value);
  else return f32_to_fp16(value);
}

// ------------------------------------------------------------ value vector

// N consecutive fp32 values; every operator rounds once per element, so a
// straight-line program evaluated on Vec<N> rounds exactly as on float.
template <int N>
struct Vec {
  float v[N];

  __device__ __forceinline__ Vec operator+(const Vec& o) const {
    Vec r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = v[i] + o.v[i];
    return r;
  }
  __device__ __forceinline__ Vec operator-(const Vec& o) const {
    Vec r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = v[i] - o.v[i];
    return r;
  }
  __device__ __forceinline__ Vec operator-() const {
    Vec r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = -v[i];
    return r;
  }
  __device__ __forceinline__ Vec operator*(float k) const {
    Vec r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = v[i] * k;
    return r;
  }
  __device__ __forceinline__ static Vec zero() {
    Vec r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.v[i] = 0.0f;
    return r;
  }
};

// ------------------------------------------------- 16-bit vector memory ops

// N 16-bit elements as one 2/4/8/16-byte access (N = 1, 2, 4, 8).
template <int N> struct Raw16;
template <> struct Raw16<1> { typedef uint16_t type; };
template <> struct Raw16<2> { typedef uint32_t type; };
template <> struct Raw16<4> { typedef uint2 type; };
template <> struct Raw16<8> { typedef uint4 type; };

template <int N>
__device__ __forceinline__ void load16(const uint16_t* p, uint16_t (&out)[N]) {
  typedef typename Raw16<N>::type R;
  const R raw = *reinterpret_cast<const R*>(p);
  __builtin_memcpy(out, &raw, sizeof(R));
}

template <int N>
__device__ __forceinline__ void store16(uint16_t* p, const uint16_t (&in)[N]) {
  typedef typename Raw16<N>::type R;
  R raw;
  __builtin_memcpy(&raw, in, sizeof(R));
  *reinterpret_cast<R*>(p) = raw;
}

// Streaming forms of the same accesses: the instruction carries the
// non-temporal hint (`nt`), so data touched once does not displace reusable
// lines in L2 and the Infinity Cache. The builtins take scalar and
// ext_vector_type operands, hence these twins of Raw16. Whether a hint pays
// depends on what the neighbouring kernels read, so each use was measured
// inside the plans, not in isolation (where streamed plane stores looked 40 %
// faster but ran 10-20 % slower in the plans).
template <int N> struct Stream16;
template <> struct Stream16<1> { typedef uint16_t type; };
template <> struct Stream16<2> { typedef uint32_t type; };
template <> struct Stream16<4> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct Stream16<8> { typedef uint32_t type __attribute__((ext_vector_type(4))); };

template <int N>
__device__ __forceinline__ void store16_stream(uint16_t* p, const uint16_t (&in)[N]) {
  typedef typename Stream16<N>::type R;
  R raw;
  __builtin_memcpy(&raw, in, sizeof(R));
  __builtin_nontemporal_store(raw, reinterpret_cast<R*>(p));
}

// N 16-bit elements as raw bits (Raw16's layout), loaded with the
// non-temporal hint.
template <int N>
__device__ __forceinline__ typename Raw16<N>::type load_raw16_stream(const uint16_t* p) {
  typedef typename Stream16<N>::type R;
  const R bits = __builtin_nontemporal_load(reinterpret_cast<const R*>(p));
  typename Raw16<N>::type raw;
  __builtin_memcpy(&raw, &bits, sizeof(raw));
  return raw;
}

// N 16-bit elements held as raw bits -> fp32.
template <int kDType, int N>
__device__ __forceinline__ Vec<N> raw_to_vec(const typename Raw16<N>::type& bits) {
  uint16_t raw[N];
  __builtin_memcpy(raw, &bits, sizeof(bits));
  Vec<N> r;
#pragma unroll
  for (int i = 0; i < N; ++i) r.v[i] = to_f32<kDType>(raw[i]);
  return r;
}

template <int kDType, int N>
__device__ __forceinline__ Vec<N> load_vec(const uint16_t* p) {
  uint16_t raw[N];
  load16<N>(p, raw);
  Vec<N> r;
#pragma unroll
  for (int i = 0; i < N; ++i) r.v[i] = to_f32<kDType>(raw[i]);
  return r;
}

// kStream: store with the non-temporal hint (data nobody reads back soon).
template <int kDType, int N, bool kStream = false>
__device__ __forceinline__ void store_vec(uint16_t* p, const Vec<N>& value) {
  uint16_t raw[N];
#pragma unroll
  for (int i = 0; i < N; ++i) raw[i] = from_f32<kDType>(value.v[i]);
  if constexpr (kStream) {
    store16_stream<N>(p, raw);
  } else {
    store16<N>(p, raw);
  }
}

}  // namespace fastmm

#endif  // FASTMM_DEVICE_H
