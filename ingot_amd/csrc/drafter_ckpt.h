// A DFlash2 drafter checkpoint read into host memory (loader.cpp), from which drafter.hip builds the drafter: the
// description, every projection as an MLX int4 g64 matrix (quantized at load when the file holds bf16 weights, as
// DFlash2Drafter does: Sources/Ingot/Drafter.swift:160-172), the norms, the conv taps and the selector's codebooks.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ih_internal.h"

namespace ih {

// An MLX int4 g64 matrix [N, K]: words [N][K/8] (low nibble first), bf16 scales and biases [N][K/64].
struct HostQ4 {
  int N = 0, K = 0;
  std::vector<uint32_t> w;
  std::vector<uint16_t> s, b;
  // Rows [r0, r0 + n) of this matrix (the k|v rows of q|k|v).
  HostQ4 rows(int r0, int n) const;
  // Rows of `o` appended (the concatenation of q, k and v, or gate and up).
  void append(const HostQ4& o);
};

struct DrafterLayerCkpt {
  std::vector<uint16_t> n1, n2, qn, kn;  // bf16 [H], [H], [HD], [HD]
  std::vector<uint16_t> abase, mbase;    // bf16 [2 (prep|finish)][2 (tap)][H] (DFlash2 only)
  HostQ4 qkv, o, gu, down, aproj, mproj;  // q|k|v and gate|up concatenated by rows
};

struct DrafterCkpt {
  ih_drafter_desc d{};
  std::vector<DrafterLayerCkpt> layers;
  HostQ4 fc, hproj;                     // hproj: DFlash2's candidate_selector.hidden_projection
  std::vector<uint16_t> hnorm, fnorm;   // bf16 [H]
  std::vector<uint16_t> pred, succ;     // bf16 [V][rank] (DFlash2)
};

// Reads a drafter directory (config.json with dflash_config + safetensors) for a target of description `t`.
int read_drafter_mlx(const std::string& dir, const ih_model_desc& t, DrafterCkpt& out);

// MLX affine quantization of one [N, K] bf16 matrix to 4 bits in groups of 64 (DenseQ.quantizeAffine,
// Sources/Ingot/Layers/Linear.swift:592-628).
void quantize_int4_g64(const uint16_t* src, int N, int K, HostQ4& out);

}  // namespace ih
