#pragma once
// The weight-tensor view that appears in Backend signatures. Same enumerators (ggml type ids) and fields as the
// reference's nibble::Tensor (src/tensor.h:21-66) so that Backend implementations are interchangeable; the HIP
// backend runs no weight ops yet and only needs the type to exist.
#include <array>
#include <cstdint>

namespace nibble {

enum class DType : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

// Non-owning view of a contiguous row-major tensor: ne[1] rows of ne[0] elements.
struct Tensor {
  DType type = DType::F32;
  int n_dims = 0;
  std::array<int64_t, 4> ne{1, 1, 1, 1};
  const void* data = nullptr;
  int64_t rows() const { return ne[1] * ne[2] * ne[3]; }
};

}  // namespace nibble
