// Boundary tensor of the domain runtime interface (the reference's
// include/hcp_ringattn/core/tensor_types.h:9-27): a named host-memory tensor.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace hcp_ringattn {

enum class TensorDType { kUnknown = 0, kFloat16 = 1, kBFloat16 = 2, kFloat32 = 3, kInt32 = 4, kInt64 = 5 };

struct BoundaryTensor {
  std::string name;
  TensorDType dtype = TensorDType::kUnknown;
  std::string layout;
  std::vector<int64_t> shape;
  std::vector<uint8_t> payload;  // host bytes, row-major in `shape`
};

}  // namespace hcp_ringattn
