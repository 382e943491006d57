// The int8 Linear stack of one Ovi / Wan2.2 DiT block on the GPU.
//
// Reference: OviDit::load_impl (src/model/ovi_dit.cpp:505-530) names and
// checks the block's Linears; the block forward (ovi_dit.cpp:176-259) runs
// them through mlin:
//   self_attn  q, k, v on the modulated norm1 output; o on the attention
//              output, then x += o * e[2]   (self_attn_fwd 176-188, block_self_fwd 205-212)
//   cross_attn q on the tokens; k, v on the text context; in fusion layers
//              k_fusion, v_fusion on the normed other-branch tokens; o on the
//              summed attention outputs, then x += o  (fusion_cross_ffn, 229-256)
//   ffn        fc1 (ffn.0) + GELU-tanh, fc2 (ffn.2), then x += fc2 * e[5]
//                                                     (ffn_fwd, 214-222)
// Linears that read the same input run as one GEMM, concatenated along out
// (q|k|v, cross k|v, k_fusion|v_fusion): bit-identical to separate mlin calls
// (activation quantization is per input row; each output column depends only
// on its own weight row and scale). Everything between the Linears (norms,
// modulation, RoPE, attention) is outside this path: those tensors are
// inputs here, device-resident; except that the norm + modulation in front
// of q|k|v and of fc1 can be folded into their activation quantizers
// (shift_sa/scale_sa, shift_ffn/scale_ffn below: then h_sa / h_ffn are not
// read and x itself is normalized, bit-exact with the reference build).
#pragma once
#include <array>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "sd/qlinear.h"
#include "sd/tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

// Device pointers for one block's linear stack (all F32 row-major).
typedef struct sd_dit_block_io {
  int64_t M;             // tokens of this branch
  int64_t Mc;            // text context rows
  int64_t Mt;            // other-branch rows (fusion layers; 0 = none)
  const float* h_sa;     // [M,dim]   input of q|k|v
  const float* att;      // [M,dim]   self-attention output, input of o
  const float* gate_sa;  // [dim]     e[2]
  const float* xq;       // [M,dim]   input of cross q
  const float* ctx;      // [Mc,dim]  input of cross k|v
  const float* tn;       // [Mt,dim]  input of k_fusion|v_fusion
  const float* xt;       // [M,dim]   cross attention output sum, input of cross o
  const float* h_ffn;    // [M,dim]   input of fc1
  const float* gate_ffn; // [dim]     e[5]
  float* qkv;            // [M,3dim]  out
  float* cq;             // [M,dim]   out
  float* ckv;            // [Mc,2dim] out
  float* kvt;            // [Mt,2dim] out (fusion layers)
  float* hid;            // [M,ffn]   out: gelu_tanh(fc1)
  float* x;              // [M,dim]   residual stream, updated in place
  // Optional (NULL = use h_sa / h_ffn): the modulation rows e[0], e[1]
  // ([dim] shift, scale) of norm1 and e[3], e[4] of norm2; q|k|v then read
  // mod_rows(layernorm(x)) at block entry (ovi_dit.cpp:208-209) and fc1
  // mod_rows(layernorm(x)) after the cross-attention update (216-217).
  const float* shift_sa;
  const float* scale_sa;
  const float* shift_ffn;
  const float* scale_ffn;
  float eps;             // layernorm epsilon (the reference's kEps, 1e-6)
} sd_dit_block_io;

// One Linear's arrays for sd_dit_block_create (all host or all device).
typedef struct sd_linear {
  const int8_t* w;       // [out,in] int8
  const float* scale;    // [out]
  const float* bias;     // [out] or NULL
  int64_t out, in;
} sd_linear;

typedef struct sd_dit_block sd_dit_block;

// Order of `lin`: self q, k, v, o; cross q, k, v, o; k_fusion, v_fusion;
// ffn.0, ffn.2 (the fusion pair is ignored when fusion == 0).
int sd_dit_block_create(const sd_linear* lin, int fusion, int on_device, sd_dit_block** out);
// nblocks blocks from host arrays (lin: 12 per block, same order) in one
// streamed weight upload; out[i] receives block i.
int sd_dit_block_create_many(const sd_linear* lin, int nblocks, int fusion, sd_dit_block** out);
int sd_dit_block_forward(const sd_dit_block* b, const sd_dit_block_io* io, void* stream);
int sd_dit_block_free(sd_dit_block* b);
// 2*M*N*K summed over the block's Linears for these row counts.
double sd_dit_block_ops(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt);
// Thread-local text of the last sd_dit_block_* error.
const char* sd_dit_last_error(void);

#ifdef __cplusplus
}

namespace sd {
namespace gpu {

class DitBlock {
 public:
  enum Lin { Q, K, V, O, CQ, CK, CV, CO, KF, VF, FC1, FC2, kCount };
  // lin[Lin] = the block's Linears (host or device arrays).
  DitBlock(const LinearPart (&lin)[kCount], bool fusion, bool on_device);
  // Many blocks from host arrays in one streamed weight upload
  // (QLinear::upload_many).
  static std::vector<DitBlock> create_many(const std::vector<std::array<LinearPart, kCount>>& blocks,
                                           bool fusion);
  int64_t dim() const { return dim_; }
  int64_t ffn_dim() const { return ffn_; }
  bool fusion() const { return fusion_; }
  // Runs the linear stack, stream-ordered (throws std::runtime_error).
  void forward_linears(const sd_dit_block_io& io, void* stream) const;
  double ops(int64_t M, int64_t Mc, int64_t Mt) const;

 private:
  DitBlock() = default;
  static void check_shapes(const LinearPart* l, bool fusion);
  QLinear qkv_, o_, cq_, ckv_, kvf_, co_, fc1_, fc2_;
  int64_t dim_ = 0, ffn_ = 0;
  bool fusion_ = false;
};

// Block `layer` of a backbone in a load_sdcpp map, with the names and checks
// of OviDit::load_impl (ovi_dit.cpp:505-530): "<prefix>blocks.<layer>.
// self_attn.{q,k,v,o}", "cross_attn.{q,k,v,o}", "cross_attn.{k_fusion,
// v_fusion}" (fusion layers), "ffn.0", "ffn.2". prefix is "video_model." or
// "audio_model.".
DitBlock dit_block_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                             const std::string& prefix, int layer, int64_t dim, int64_t ffn_dim,
                             bool fusion);
// Blocks `layers` of a backbone, all uploaded in one stream (the pack's
// int8 views are copied through pinned buffers while the GPU repacks).
std::vector<DitBlock> dit_blocks_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                                           const std::string& prefix,
                                           const std::vector<int>& layers, int64_t dim,
                                           int64_t ffn_dim, bool fusion);

}  // namespace gpu
}  // namespace sd
#endif
