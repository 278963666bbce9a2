#pragma once

#include <concepts>

namespace sil {

// Element types an array may hold: the same set as the reference
// (include/types.h:7-9); float is the type the GPU path computes in.
template <typename T>
concept value_type = std::same_as<T, float> || std::same_as<T, int> || std::same_as<T, bool>;

}  // namespace sil
