// PyTorch-ROCm operators over the C ABI of libfastmm_amd.so.
//
// Two operator namespaces:
//
//   rdna3_fastmm::linear, ::linear_rank7, ::linear_rank48
//       The allocating F.linear operators, with the reference's schemas
//       (src/rdna3_fastmm/linear.py:50-167: functional, `(Tensor input,
//       Tensor weight, Tensor? bias=None) -> Tensor`, any number of leading
//       dimensions). The whole call runs here: the transformed planes and the
//       products are allocated on the input's device, the planes (and the
//       split-K scratch) are released before the output is allocated, as the
//       reference does (linear.py:66-153), and every stage is one C-ABI launch
//       on the current HIP stream.
//
//   rdna3_fastmm_hip::left_transform, ::weight_transform, ::right_transform,
//   ::leaf_products, ::leaf_scratch_bytes, ::reconstruct
//       One operator per C-ABI entry point, writing into caller tensors; the
//       plans (rdna3_fastmm.runtime) call these.
//
// Argument errors raise ValueError (TORCH_CHECK_VALUE) before any launch; a
// status from the library raises RuntimeError with fastmm_last_error(). There
// is no fallback: without a GPU the library reports the failed launch.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <optional>
#include <vector>

#include "fastmm_amd.h"

namespace {

int dtype_code(at::ScalarType type) {
  switch (type) {
    case at::kBFloat16: return FASTMM_BF16;
    case at::kHalf: return FASTMM_FP16;
    case at::kFloat: return FASTMM_FP32;
    default: TORCH_CHECK_VALUE(false, "fastmm: unsupported element type ", type);
  }
  return -1;  // not reached
}

void check_status(int status, const char* entry) {
  TORCH_CHECK(status == FASTMM_OK, entry, " failed (", status, "): ", fastmm_last_error());
}

void* stream_of(const at::Tensor& tensor) {
  return c10::hip::getCurrentHIPStream(tensor.device().index()).stream();
}

// ceil(a / b) for b > 0; 0 for a <= 0
int64_t ceil_div(int64_t a, int64_t b) { return a > 0 ? (a - 1) / b + 1 : 0; }

// Buffer shape of a transformed operand (rows = Mb or Nb): K-slab-major
// [R, Kb/32, rows, 32] when Kb % 32 == 0, else row-major [R, rows, Kb].
std::vector<int64_t> operand_shape(int64_t rank, int64_t rows, int64_t inner) {
  if (inner % 32 == 0) return {rank, inner / 32, rows, 32};
  return {rank, rows, inner};
}

// ---------------------------------------------------------------- stage ops
//
// The library sees bare pointers, so each stage operator first checks every
// tensor against the dimensions it is given: on the first operand's ROCm
// device, contiguous, and holding at least the elements the launch reads or
// writes. A dimension that is not positive skips the count and reaches the
// library, which rejects it before any launch.

// Elements a launch over these extents covers (0 when one is not positive).
int64_t covered(const char* op, std::initializer_list<int64_t> extents) {
  for (int64_t e : extents)
    if (e < 1) return 0;
  int64_t n = 1;
  for (int64_t e : extents)
    TORCH_CHECK_VALUE(!__builtin_mul_overflow(n, e, &n), op, ": dimensions too large");
  return n;
}

void require_buffer(const char* op, const char* name, const at::Tensor& tensor, const at::Device& device,
                    int64_t elements) {
  TORCH_CHECK_VALUE(tensor.device().is_cuda() && tensor.device() == device, op, ": ", name,
                    " must be on the operands' ROCm device (", device, "), got ", tensor.device());
  TORCH_CHECK_VALUE(tensor.is_contiguous(), op, ": ", name, " must be contiguous");
  TORCH_CHECK_VALUE(tensor.numel() >= elements, op, ": ", name, " holds ", tensor.numel(),
                    " elements, the launch covers ", elements);
}

struct SchemeDims {
  int64_t size, rank;
};

SchemeDims scheme_dims(int64_t scheme) {
  int s = 0, rank = 0;
  check_status(fastmm_scheme_info(static_cast<int>(scheme), &s, &rank), "fastmm_scheme_info");
  return {s, rank};
}

// Source [rows, inner] (or [inner, columns]) and planes [R, ceil(a/s), ceil(b/s)].
void check_transform(const char* op, int64_t scheme, const at::Tensor& source, const at::Tensor& planes,
                     int64_t a, int64_t b) {
  TORCH_CHECK_VALUE(source.device().is_cuda(), op, ": tensors must be on a ROCm device, got ", source.device());
  const SchemeDims d = scheme_dims(scheme);
  require_buffer(op, "source", source, source.device(), covered(op, {a, b}));
  require_buffer(op, "planes", planes, source.device(),
                 covered(op, {d.rank, ceil_div(a, d.size), ceil_div(b, d.size)}));
}

void left_transform(int64_t scheme, const at::Tensor& input, const at::Tensor& output, int64_t rows,
                    int64_t inner) {
  check_transform("rdna3_fastmm_hip::left_transform", scheme, input, output, rows, inner);
  c10::DeviceGuard guard(input.device());
  check_status(fastmm_left_transform(static_cast<int>(scheme), dtype_code(input.scalar_type()),
                                     dtype_code(output.scalar_type()), input.data_ptr(), output.data_ptr(), rows,
                                     inner, stream_of(input)),
               "fastmm_left_transform");
}

void weight_transform(int64_t scheme, const at::Tensor& weight, const at::Tensor& output, int64_t columns,
                      int64_t inner) {
  check_transform("rdna3_fastmm_hip::weight_transform", scheme, weight, output, columns, inner);
  c10::DeviceGuard guard(weight.device());
  check_status(fastmm_weight_transform(static_cast<int>(scheme), dtype_code(weight.scalar_type()),
                                       dtype_code(output.scalar_type()), weight.data_ptr(), output.data_ptr(),
                                       columns, inner, stream_of(weight)),
               "fastmm_weight_transform");
}

void right_transform(int64_t scheme, const at::Tensor& right, const at::Tensor& output, int64_t inner,
                     int64_t columns) {
  check_transform("rdna3_fastmm_hip::right_transform", scheme, right, output, inner, columns);
  c10::DeviceGuard guard(right.device());
  check_status(fastmm_right_transform(static_cast<int>(scheme), dtype_code(right.scalar_type()),
                                      dtype_code(output.scalar_type()), right.data_ptr(), output.data_ptr(), inner,
                                      columns, stream_of(right)),
               "fastmm_right_transform");
}

void leaf_products(int64_t rank, const at::Tensor& left, const at::Tensor& right, const at::Tensor& products,
                   int64_t block_rows, int64_t block_inner, int64_t block_columns,
                   const std::optional<at::Tensor>& scratch) {
  const char* op = "rdna3_fastmm_hip::leaf_products";
  TORCH_CHECK_VALUE(left.device().is_cuda(), op, ": tensors must be on a ROCm device, got ", left.device());
  TORCH_CHECK_VALUE(right.scalar_type() == left.scalar_type(), op, ": left and right planes differ in dtype");
  require_buffer(op, "left planes", left, left.device(), covered(op, {rank, block_rows, block_inner}));
  require_buffer(op, "right planes", right, left.device(), covered(op, {rank, block_columns, block_inner}));
  require_buffer(op, "products", products, left.device(), covered(op, {rank, block_rows, block_columns}));
  if (scratch.has_value()) require_buffer(op, "scratch", *scratch, left.device(), 0);
  c10::DeviceGuard guard(left.device());
  void* scratch_data = scratch.has_value() ? scratch->data_ptr() : nullptr;
  const int64_t scratch_bytes = scratch.has_value() ? scratch->numel() * scratch->element_size() : 0;
  check_status(fastmm_leaf_products(static_cast<int>(rank), dtype_code(left.scalar_type()), left.data_ptr(),
                                    right.data_ptr(), products.data_ptr(), dtype_code(products.scalar_type()),
                                    block_rows, block_inner, block_columns, scratch_data, scratch_bytes,
                                    stream_of(left)),
               "fastmm_leaf_products");
}

int64_t leaf_scratch_bytes(int64_t rank, at::ScalarType operand_type, at::ScalarType products_type,
                           int64_t block_rows, int64_t block_inner, int64_t block_columns, at::Device device) {
  c10::DeviceGuard guard(device);
  int64_t bytes = 0;
  check_status(fastmm_leaf_scratch_bytes(static_cast<int>(rank), dtype_code(operand_type), dtype_code(products_type),
                                         block_rows, block_inner, block_columns, &bytes),
               "fastmm_leaf_scratch_bytes");
  return bytes;
}

void reconstruct(int64_t scheme, const at::Tensor& products, const std::optional<at::Tensor>& bias,
                 const at::Tensor& output, int64_t rows, int64_t columns) {
  const char* op = "rdna3_fastmm_hip::reconstruct";
  TORCH_CHECK_VALUE(products.device().is_cuda(), op, ": tensors must be on a ROCm device, got ", products.device());
  const SchemeDims d = scheme_dims(scheme);
  require_buffer(op, "products", products, products.device(),
                 covered(op, {d.rank, ceil_div(rows, d.size), ceil_div(columns, d.size)}));
  require_buffer(op, "output", output, products.device(), covered(op, {rows, columns}));
  if (bias.has_value()) {
    TORCH_CHECK_VALUE(bias->scalar_type() == output.scalar_type(), op, ": bias must have the output's dtype");
    require_buffer(op, "bias", *bias, products.device(), covered(op, {columns}));
  }
  c10::DeviceGuard guard(products.device());
  check_status(fastmm_reconstruct(static_cast<int>(scheme), dtype_code(products.scalar_type()), products.data_ptr(),
                                  bias.has_value() ? bias->data_ptr() : nullptr, dtype_code(output.scalar_type()),
                                  output.data_ptr(), rows, columns, stream_of(products)),
               "fastmm_reconstruct");
}

// ------------------------------------------------------ allocating F.linear

void check_operands(const char* name, const at::Tensor& input, const at::Tensor& weight,
                    const std::optional<at::Tensor>& bias) {
  TORCH_CHECK_VALUE((input.scalar_type() == at::kBFloat16 || input.scalar_type() == at::kHalf) &&
                        weight.scalar_type() == input.scalar_type(),
                    name, " needs bf16 or fp16 input and weight of one dtype");
  TORCH_CHECK_VALUE(input.device().is_cuda() && weight.device() == input.device(), name,
                    " needs input and weight on one ROCm device");
  TORCH_CHECK_VALUE(weight.dim() == 2 && input.dim() >= 1 && input.size(-1) == weight.size(1), name,
                    ": input [..., K] and weight [N, K] do not match");
  TORCH_CHECK_VALUE(input.is_contiguous() && weight.is_contiguous(), name, " needs contiguous input and weight");
  if (bias.has_value()) {
    const at::Tensor& b = *bias;
    TORCH_CHECK_VALUE(b.dim() == 1 && b.size(0) == weight.size(0) && b.scalar_type() == input.scalar_type() &&
                          b.device() == input.device() && b.is_contiguous(),
                      name, ": bias must be a contiguous [N] tensor of the input dtype");
  }
}

at::Tensor linear_through(int scheme_id, const char* name, const at::Tensor& input, const at::Tensor& weight,
                          const std::optional<at::Tensor>& bias) {
  check_operands(name, input, weight, bias);
  int s = 0, rank = 0;
  check_status(fastmm_scheme_info(scheme_id, &s, &rank), "fastmm_scheme_info");
  c10::DeviceGuard guard(input.device());
  const int64_t inner = input.size(-1), columns = weight.size(0);
  const at::Tensor flat = input.reshape({-1, inner});
  const int64_t rows = flat.size(0);
  TORCH_CHECK_VALUE(rows > 0 && inner > 0 && columns > 0, name, ": empty input or weight");
  const int64_t mb = ceil_div(rows, s), kb = ceil_div(inner, s), nb = ceil_div(columns, s);
  const auto planes = input.options().dtype(at::kHalf);
  at::Tensor left = at::empty(operand_shape(rank, mb, kb), planes);
  at::Tensor right = at::empty(operand_shape(rank, nb, kb), planes);
  left_transform(scheme_id, flat, left, rows, inner);
  weight_transform(scheme_id, weight, right, columns, inner);
  at::Tensor products = at::empty({rank, mb, nb}, planes);
  const int64_t scratch_bytes = leaf_scratch_bytes(rank, at::kHalf, at::kHalf, mb, kb, nb, input.device());
  std::optional<at::Tensor> scratch;
  if (scratch_bytes > 0) scratch = at::empty({scratch_bytes}, input.options().dtype(at::kByte));
  leaf_products(rank, left, right, products, mb, kb, nb, scratch);
  left.reset();  // the planes and the scratch go back to the allocator before the output exists
  right.reset();
  scratch.reset();
  at::Tensor output = at::empty({rows, columns}, input.options());
  reconstruct(scheme_id, products, bias, output, rows, columns);
  std::vector<int64_t> shape(input.sizes().begin(), input.sizes().end());
  shape.back() = columns;
  return output.view(shape);
}

at::Tensor linear_rank49(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias) {
  return linear_through(FASTMM_SCHEME_RANK49, "rdna3_fastmm::linear", input, weight, bias);
}

at::Tensor linear_rank7(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias) {
  return linear_through(FASTMM_SCHEME_RANK7, "rdna3_fastmm::linear_rank7", input, weight, bias);
}

at::Tensor linear_rank48(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias) {
  return linear_through(FASTMM_SCHEME_RANK48, "rdna3_fastmm::linear_rank48", input, weight, bias);
}

}  // namespace

TORCH_LIBRARY(rdna3_fastmm, m) {
  m.def("linear(Tensor input, Tensor weight, Tensor? bias=None) -> Tensor");
  m.def("linear_rank7(Tensor input, Tensor weight, Tensor? bias=None) -> Tensor");
  m.def("linear_rank48(Tensor input, Tensor weight, Tensor? bias=None) -> Tensor");
}

// CompositeExplicitAutograd: one kernel for every device, so an input on the
// wrong device gets the operators' own ValueError; shape inference for fake
// tensors is registered from Python.
TORCH_LIBRARY_IMPL(rdna3_fastmm, CompositeExplicitAutograd, m) {
  m.impl("linear", &linear_rank49);
  m.impl("linear_rank7", &linear_rank7);
  m.impl("linear_rank48", &linear_rank48);
}

TORCH_LIBRARY(rdna3_fastmm_hip, m) {
  m.def("left_transform(int scheme, Tensor input, Tensor(a!) output, int rows, int inner) -> ()");
  m.def("weight_transform(int scheme, Tensor weight, Tensor(a!) output, int columns, int inner) -> ()");
  m.def("right_transform(int scheme, Tensor right, Tensor(a!) output, int inner, int columns) -> ()");
  m.def(
      "leaf_products(int rank, Tensor left, Tensor right, Tensor(a!) products, int block_rows, int block_inner, "
      "int block_columns, Tensor(b!)? scratch=None) -> ()");
  // no tensor arguments: one kernel for every dispatch key
  m.def(
      "leaf_scratch_bytes(int rank, ScalarType operand_dtype, ScalarType products_dtype, int block_rows, "
      "int block_inner, int block_columns, Device device) -> int",
      &leaf_scratch_bytes);
  m.def("reconstruct(int scheme, Tensor products, Tensor? bias, Tensor(a!) output, int rows, int columns) -> ()");
}

TORCH_LIBRARY_IMPL(rdna3_fastmm_hip, CompositeExplicitAutograd, m) {
  m.impl("left_transform", &left_transform);
  m.impl("weight_transform", &weight_transform);
  m.impl("right_transform", &right_transform);
  m.impl("leaf_products", &leaf_products);
  m.impl("reconstruct", &reconstruct);
}

