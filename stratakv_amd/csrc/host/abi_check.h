// abi_check.h -- turn C ABI status codes into the reference's exception
// types: SKV_ERR_INVALID_ARGUMENT -> std::invalid_argument, anything else ->
// std::runtime_error (the reference's CUDA-failure convention,
// src/memory/block_pool.cpp:36-40).
#pragma once

#include <stdexcept>
#include <string>

#include "stratakv_amd.h"

namespace stratakv {
namespace detail {

inline void check(int status, const char* what) {
    if (status == SKV_OK) return;
    const std::string msg = std::string(what) + ": " + skv_last_error();
    if (status == SKV_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

}  // namespace detail
}  // namespace stratakv
