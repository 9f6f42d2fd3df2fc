// activation_quant.hpp — C++ counterpart of the reference module
// candelora_metal_kernels::activation_quant (src/activation_quant.rs:7-44).
#pragma once

namespace candelora {

// ActivationQuantMode (src/activation_quant.rs:7-21); default Off.
enum class ActivationQuantMode {
  Off,   // keep floating-point activations
  W8A8,  // per-row int8 fake quantisation of the activations
  W4A8,  // contract only: runs as Off unless `strict`
};

// ActivationQuantConfig (src/activation_quant.rs:23-44).
struct ActivationQuantConfig {
  ActivationQuantMode mode = ActivationQuantMode::Off;
  bool strict = false;

  bool is_enabled() const { return mode != ActivationQuantMode::Off; }
};

inline const char* to_string(ActivationQuantMode m) {
  switch (m) {
    case ActivationQuantMode::Off: return "Off";
    case ActivationQuantMode::W8A8: return "W8A8";
    default: return "W4A8";
  }
}

}  // namespace candelora
