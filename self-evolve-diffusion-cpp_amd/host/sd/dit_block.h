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

#include "sd/pack.h"
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

// The block's normalization vectors, [dim] F32 host arrays each (copied by
// sd_dit_block_set_norms). Names of OviDit::load_impl (ovi_dit.cpp:509-537).
typedef struct sd_dit_norms {
  const float* sa_nq;      // self_attn.norm_q.weight
  const float* sa_nk;      // self_attn.norm_k.weight
  const float* ca_nq;      // cross_attn.norm_q.weight
  const float* ca_nk;      // cross_attn.norm_k.weight
  const float* ln3_w;      // norm3.weight   (used by non-fusion blocks)
  const float* ln3_b;      // norm3.bias
  const float* nk_fusion;  // cross_attn.norm_k_fusion.weight        (fusion blocks)
  const float* pnf_w;      // cross_attn.pre_attn_norm_fusion.weight (fusion blocks)
  const float* pnf_b;      // cross_attn.pre_attn_norm_fusion.bias   (fusion blocks)
} sd_dit_norms;

// One whole block forward on device arrays (sd_dit_block_step_forward).
typedef struct sd_dit_block_step {
  int64_t M;             // tokens of this branch
  int64_t Mc;            // text context rows (> 0)
  int64_t Mt;            // target rows (fusion blocks: the other branch)
  int heads;             // attention heads; head_dim = dim/heads must be 128
  float eps;             // the reference's kEps (1e-6)
  float* x;              // [M,dim] residual stream, updated in place
  const float* ctx;      // [Mc,dim] text context (embed_ctx output)
  const float* target;   // [Mt,dim] other branch's tokens (fusion blocks)
  const float* e;        // [6,dim] modulation rows (time rows + ModulationAdd)
  const float* cs;       // [M,nr,2] RoPE (cos, sin) of this branch (sd_rope_table_*)
  int nr;                // pairs rotated per head (64 video, 22 audio)
  const float* cs_tgt;   // [Mt,nr_tgt,2] RoPE table of the target branch (fusion)
  int nr_tgt;
  void* ws;              // device workspace, sd_dit_block_workspace_bytes bytes
  size_t ws_bytes;
} sd_dit_block_step;

// Phases of sd_dit_block_step_forward: the self-attention branch
// (block_self_fwd, ovi_dit.cpp:205-212) and the cross attention + FFN
// (block_vanilla_fwd's rest, 259-268, or fusion_cross_ffn, 229-256).
enum { SD_DIT_SELF = 1, SD_DIT_CROSS_FFN = 2, SD_DIT_ALL = 3 };

// Order of `lin`: self q, k, v, o; cross q, k, v, o; k_fusion, v_fusion;
// ffn.0, ffn.2 (the fusion pair is ignored when fusion == 0).
int sd_dit_block_create(const sd_linear* lin, int fusion, int on_device, sd_dit_block** out);
// nblocks blocks from host arrays (lin: 12 per block, same order) in one
// streamed weight upload; out[i] receives block i.
int sd_dit_block_create_many(const sd_linear* lin, int nblocks, int fusion, sd_dit_block** out);
int sd_dit_block_forward(const sd_dit_block* b, const sd_dit_block_io* io, void* stream);
// The linear stacks of two blocks whose inputs do not depend on each other
// (the video and audio blocks of one twin layer, each with its own io): the
// same results as sd_dit_block_forward on each, with the attention Linears
// of both and the two cross-attention output projections each run as one
// grouped launch (sdq_qlinear_group) when no output overlaps another input.
int sd_dit_block_forward_pair(const sd_dit_block* a, const sd_dit_block_io* ia,
                              const sd_dit_block* b, const sd_dit_block_io* ib, void* stream);
// The same on two streams, forked from `stream` and joined back into it
// (sdq_stream_wait): a's own Linears on `stream`; b's, and a's text k|v and
// fusion k|v, on stream2 (a balanced split when a is the longer branch).
// When the two sides would touch each other's outputs, or stream2 is NULL
// or equal to stream: as sd_dit_block_forward_pair. Same results.
int sd_dit_block_forward_pair2(const sd_dit_block* a, const sd_dit_block_io* ia,
                               const sd_dit_block* b, const sd_dit_block_io* ib, void* stream,
                               void* stream2);
int sd_dit_block_free(sd_dit_block* b);
// Copies the block's norm vectors to the device (required before
// sd_dit_block_step_forward; the fusion ones for fusion blocks, ln3 for others).
int sd_dit_block_set_norms(sd_dit_block* b, const sd_dit_norms* n);
// The block's own modulation bias (modulation.modulation, [6,dim] F32 host
// array, copied), and e = t6 + that bias on the device: the per-layer
// ModulationAdd of OviDit::forward (ovi_dit.cpp:716-723, one fp32 add per
// value, bit-exact). t6 [6,dim] are the time rows (time_projection output),
// e [6,dim] receives the block's modulation rows for sd_dit_block_step_forward.
int sd_dit_block_set_modulation(sd_dit_block* b, const float* mod);
int sd_dit_block_modulation(const sd_dit_block* b, const float* t6, float* e, void* stream);
// Blocks `layers[0..n)` of backbone `prefix` ("video_model." or
// "audio_model.") of a .sdcpp file, whole: the 12 int8 Linears, the norm
// vectors and modulation.modulation, with OviDit::load_impl's names, checks
// and messages (ovi_dit.cpp:397-415, 505-537). file_reads = 1 reads the
// weights with large sequential reads into the pinned staging ring
// (sdq_weight_upload_file); 0 goes through load_sdcpp's mapping. out[i]
// receives block layers[i]; on error none is returned.
int sd_dit_blocks_from_pack(const char* path, const char* prefix, const int* layers, int n,
                            int64_t dim, int64_t ffn_dim, int fusion, int file_reads,
                            sd_dit_block** out);
// Device workspace bytes that sd_dit_block_step_forward needs for these rows.
size_t sd_dit_block_workspace_bytes(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt);
// The whole block on the GPU, stream-ordered, bit-exact with the reference
// build except the attention (split-fp16 scores, split-bf16 P.V, an online softmax:
// within 2e-5 of the reference's sdpa); phases = SD_DIT_SELF | SD_DIT_CROSS_FFN. A fusion
// layer (ovi_dit.cpp:726-734) runs SELF on both branches, then CROSS_FFN of
// the audio branch (target = video x), then of the video branch with target =
// a copy of the audio x taken before the audio CROSS_FFN.
int sd_dit_block_step_forward(const sd_dit_block* b, const sd_dit_block_step* st, int phases,
                              void* stream);
// The same block on `batch` sequences stacked along the rows, sharing the
// weights and the modulation rows e: the conditional and unconditional
// forwards of a guidance step (denoise.cpp:95-98) as one pass, each with its
// own text context. st.M, st.Mc, st.Mt are per sequence; x holds batch*M
// rows, ctx batch*Mc, target batch*Mt (sequence b at row b*M, b*Mc, b*Mt);
// cs covers batch*M rows and cs_tgt batch*Mt (each sequence's table
// repeated); ws is sd_dit_block_workspace_bytes(batch*M, batch*Mc,
// batch*Mt). Every step is per row except the attention, which stays inside
// each sequence (sdq_sdpa_batched): bit-identical to `batch` separate calls.
int sd_dit_block_step_forward_batched(const sd_dit_block* b, const sd_dit_block_step* st,
                                      int batch, int phases, void* stream);
// 2*M*N*K of the Linears plus the attention products (4*Lq*Lk*dim per sdpa).
double sd_dit_block_step_ops(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt);
// 2*M*N*K summed over the block's Linears for these row counts.
double sd_dit_block_ops(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt);
// Thread-local text of the last sd_dit_block_* error.
const char* sd_dit_last_error(void);

#ifdef __cplusplus
}

namespace sd {
namespace gpu {

struct LinCall;  // one Linear of a grouped run (dit_block.cpp)

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
  friend void forward_linears_pair(const DitBlock& a, const sd_dit_block_io& ia,
                                   const DitBlock& b, const sd_dit_block_io& ib, void* stream,
                                   void* stream2);
  double ops(int64_t M, int64_t Mc, int64_t Mt) const;
  // The whole block (norms, RoPE, attention and Linears) on device arrays.
  void set_norms(const sd_dit_norms& n);
  // modulation.modulation ([6,dim], host) and e = t6 + it on the device.
  void set_modulation(const float* mod);
  bool has_modulation() const { return static_cast<bool>(mod_); }
  void modulation_rows(const float* t6, float* e, void* stream) const;
  size_t workspace_bytes(int64_t M, int64_t Mc, int64_t Mt) const;
  // batch > 1: that many sequences stacked along the rows (see
  // sd_dit_block_step_forward_batched).
  void forward_step(const sd_dit_block_step& st, int phases, void* stream, int batch = 1) const;
  double step_ops(int64_t M, int64_t Mc, int64_t Mt) const;

 private:
  DitBlock() = default;
  static void check_shapes(const LinearPart* l, bool fusion);
  enum Norm { SA_NQ, SA_NK, CA_NQ, CA_NK, LN3_W, LN3_B, NK_F, PNF_W, PNF_B, kNorms };
  const float* norm(Norm n) const { return norms_.get() + n * dim_; }
  void self_phase(const sd_dit_block_step& st, int batch, float* ws, void* s) const;
  void check_io(const sd_dit_block_io& io) const;
  void qkv_lnmod(const sd_dit_block_io& io, void* s) const;
  void attn_linears(const sd_dit_block_io& io, std::vector<LinCall>& out) const;
  void ffn_linears(const sd_dit_block_io& io, void* s) const;
  bool ffn_item(const sd_dit_block_io& io, sdq_ffn_item* f) const;
  void cross_ffn_phase(const sd_dit_block_step& st, int batch, float* ws, void* s) const;
  friend std::vector<DitBlock> dit_blocks_from_pack_file(const std::string&, const std::string&,
                                                         const std::vector<int>&, int64_t,
                                                         int64_t, bool);
  QLinear qkv_, o_, cq_, ckv_, kvf_, co_, fc1_, fc2_;
  DeviceFloats norms_, mod_;
  int64_t dim_ = 0, ffn_ = 0;
  bool fusion_ = false;
};

// Both blocks' forward_linears (independent inputs), their attention Linears
// and cross-attention output projections grouped (sd_dit_block_forward_pair);
// with stream2 (not stream), b's Linears and a's text / fusion k|v run
// there, forked and joined (sd_dit_block_forward_pair2).
void forward_linears_pair(const DitBlock& a, const sd_dit_block_io& ia, const DitBlock& b,
                          const sd_dit_block_io& ib, void* stream, void* stream2 = nullptr);

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
// Both also load the block's norm vectors (self_attn.norm_q/k, cross_attn.
// norm_q/k, norm3.weight/bias; fusion: cross_attn.norm_k_fusion,
// pre_attn_norm_fusion.weight/bias) and modulation.modulation [1,6,dim]
// (ovi_dit.cpp:509-537), so the blocks are ready for forward_step; packs keep
// these small tensors F32 (pack_sdcpp.py:23, numel < 65536), and an int8
// one is rejected.
std::vector<DitBlock> dit_blocks_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                                           const std::string& prefix,
                                           const std::vector<int>& layers, int64_t dim,
                                           int64_t ffn_dim, bool fusion);
// The same from the file itself: the tensor table is indexed (sd::PackIndex)
// and the weights are read with large sequential reads straight into the
// pinned staging ring (QLinear::upload_many_file), no mapping.
std::vector<DitBlock> dit_blocks_from_pack_file(const std::string& path, const std::string& prefix,
                                                const std::vector<int>& layers, int64_t dim,
                                                int64_t ffn_dim, bool fusion);

}  // namespace gpu
}  // namespace sd
#endif
