// status.h -- maps libdsd_hip.so status codes back onto the exception types
// the reference API throws (std::invalid_argument / out_of_range /
// runtime_error, include/dsd/cuda_utils.h:43-53 and the class sources).
#pragma once

#include <stdexcept>
#include <string>

#include "dsd_hip.h"

namespace dsd {
namespace detail {

inline void ThrowOnError(int status) {
  if (status == DSD_OK) return;
  const std::string message = dsd_last_error();
  switch (status) {
    case DSD_ERR_INVALID_ARGUMENT: throw std::invalid_argument(message);
    case DSD_ERR_OUT_OF_RANGE: throw std::out_of_range(message);
    default: throw std::runtime_error(message);
  }
}

}  // namespace detail
}  // namespace dsd
