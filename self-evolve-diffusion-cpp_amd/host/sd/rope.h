// RoPE (cos, sin) tables for sdq_rmsnorm_rope, built on the host.
//
// Reference: blk::rope_freqs_3d / rope_freqs_1d (src/model/blocks.cpp:46-84)
// give each token's rotation angle per complex pair; blk::apply_rope
// (blocks.cpp:86-100) takes std::cos / std::sin of those angles for every
// head. The tables here hold exactly those (cosf, sinf) values, computed once
// per token grid, so the GPU rotation needs no transcendental of its own and
// stays bit-exact with the reference.
#pragma once
#include <cstdint>
#include <vector>

#ifdef __cplusplus
extern "C" {
#endif

// Table [T*H*W][n_rot][2] (cos, sin) of rope_freqs_3d(T, H, W, head_dim,
// theta); returns n_rot (head_dim/2 for head_dim 128), or -1 on bad
// arguments. cs = NULL only returns n_rot.
int sd_rope_table_3d(int T, int H, int W, int head_dim, float theta, float* cs);
// Table [L][n_rot][2] of rope_freqs_1d(L, head_dim, theta, scaling) (audio:
// the t-axis pairs only, n_rot = (head_dim - 4*(head_dim/6))/2).
int sd_rope_table_1d(int L, int head_dim, float theta, float scaling, float* cs);

#ifdef __cplusplus
}

namespace sd {
struct RopeTable {
  std::vector<float> cs;  // [L][n_rot][2]
  int64_t L = 0;
  int n_rot = 0;
};
RopeTable rope_table_3d(int T, int H, int W, int head_dim, float theta = 10000.0f);
RopeTable rope_table_1d(int L, int head_dim, float theta = 10000.0f, float scaling = 1.0f);
}  // namespace sd
#endif
