// iq2_matmul.hpp — C++ counterpart of the reference module
// candelora_metal_kernels::iq2_matmul (src/iq2_matmul.rs:31-37, 535-670).
//
// Same names, arguments and error texts as the Rust functions; the bodies call
// the C ABI of libcmk_iq2.so (include/cmk_iq2.h) instead of the Metal dispatch
// helpers.  Launches are asynchronous on the default HIP stream, like the
// reference's command-encoder dispatch; Tensor::to_vec() synchronises.
#pragma once
#include <cstddef>

#include "candelora/activation_quant.hpp"
#include "candelora/tensor.hpp"

namespace candelora {

// Iq2MatmulVariant (src/iq2_matmul.rs:31-37).
enum class Iq2MatmulVariant { Iq2Xxs, Iq2Xs, Iq2S, Iq3S };

// Generic entry point (src/iq2_matmul.rs:536-553).  x: [K] -> [N] or [M, K] -> [M, N],
// dtype F32/F16/BF16; weight_bytes / weight_scales: contiguous U8.  Output F32.
Tensor iq2_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                  size_t out_dim, size_t in_dim, Iq2MatmulVariant variant);

// src/iq2_matmul.rs:559-591: Off -> iq2_matmul; W8A8 -> per-row int8 fake-quantised
// activations; W4A8 -> error when strict, else Off.
Tensor iq2_matmul_with_activation_quant(const Tensor& x, const Tensor& weight_bytes,
                                        const Tensor& weight_scales, size_t out_dim,
                                        size_t in_dim, Iq2MatmulVariant variant,
                                        const ActivationQuantConfig& activation_quant);

// src/iq2_matmul.rs:594-602: dense [out_dim, in_dim] F16.
Tensor iq2_dequantize_to_f16(const Tensor& weight_bytes, const Tensor& weight_scales,
                             size_t out_dim, size_t in_dim, Iq2MatmulVariant variant);

// src/iq2_matmul.rs:604-670.
Tensor iq2_xxs_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                      size_t out_dim, size_t in_dim);
Tensor iq2_xs_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                     size_t out_dim, size_t in_dim);
Tensor iq2_s_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                    size_t out_dim, size_t in_dim);
Tensor iq3_s_matmul(const Tensor& x, const Tensor& weight_bytes, const Tensor& weight_scales,
                    size_t out_dim, size_t in_dim);

// Blocks until the default stream's work is done (candle's device.synchronize()).
void synchronize();

}  // namespace candelora
