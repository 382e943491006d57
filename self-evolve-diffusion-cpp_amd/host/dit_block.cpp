// sd::gpu::DitBlock — see sd/dit_block.h.
#include "sd/dit_block.h"

#include <algorithm>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace sd {
namespace gpu {

namespace {

void need(bool ok, const std::string& msg) {
  if (!ok) throw std::runtime_error("DitBlock: " + msg);
}

}  // namespace

void DitBlock::check_shapes(const LinearPart* l, bool fusion) {
  const int64_t dim = l[Q].in, ffn = l[FC1].out;
  for (int i : {Q, K, V, O, CQ, CK, CV, CO})
    need(l[i].in == dim && l[i].out == dim, "attention Linears must be [dim,dim]");
  if (fusion) need(l[KF].in == dim && l[KF].out == dim && l[VF].in == dim && l[VF].out == dim,
                   "fusion Linears must be [dim,dim]");
  need(l[FC1].in == dim && l[FC2].in == ffn && l[FC2].out == dim, "ffn shapes");
}

std::vector<DitBlock> DitBlock::create_many(
    const std::vector<std::array<LinearPart, kCount>>& blocks, bool fusion) {
  std::vector<std::vector<LinearPart>> sets;
  for (const auto& l : blocks) {
    check_shapes(l.data(), fusion);
    sets.push_back({l[Q], l[K], l[V]});
    sets.push_back({l[O]});
    sets.push_back({l[CQ]});
    sets.push_back({l[CK], l[CV]});
    if (fusion) sets.push_back({l[KF], l[VF]});
    sets.push_back({l[CO]});
    sets.push_back({l[FC1]});
    sets.push_back({l[FC2]});
  }
  std::vector<QLinear> q = QLinear::upload_many(sets);
  std::vector<DitBlock> out;
  out.reserve(blocks.size());
  size_t j = 0;
  for (size_t b = 0; b < blocks.size(); b++) {
    DitBlock d;
    d.fusion_ = fusion;
    d.dim_ = blocks[b][Q].in;
    d.ffn_ = blocks[b][FC1].out;
    d.qkv_ = std::move(q[j++]);
    d.o_ = std::move(q[j++]);
    d.cq_ = std::move(q[j++]);
    d.ckv_ = std::move(q[j++]);
    if (fusion) d.kvf_ = std::move(q[j++]);
    d.co_ = std::move(q[j++]);
    d.fc1_ = std::move(q[j++]);
    d.fc2_ = std::move(q[j++]);
    out.push_back(std::move(d));
  }
  return out;
}

DitBlock::DitBlock(const LinearPart (&l)[kCount], bool fusion, bool on_device) : fusion_(fusion) {
  check_shapes(l, fusion);
  dim_ = l[Q].in;
  ffn_ = l[FC1].out;
  qkv_ = QLinear(std::vector<LinearPart>{l[Q], l[K], l[V]}, on_device);
  o_ = QLinear(std::vector<LinearPart>{l[O]}, on_device);
  cq_ = QLinear(std::vector<LinearPart>{l[CQ]}, on_device);
  ckv_ = QLinear(std::vector<LinearPart>{l[CK], l[CV]}, on_device);
  if (fusion) kvf_ = QLinear(std::vector<LinearPart>{l[KF], l[VF]}, on_device);
  co_ = QLinear(std::vector<LinearPart>{l[CO]}, on_device);
  fc1_ = QLinear(std::vector<LinearPart>{l[FC1]}, on_device);
  fc2_ = QLinear(std::vector<LinearPart>{l[FC2]}, on_device);
}

// One Linear of a run: out[M, N] = epilogue(A[M, K] W^T + b).
struct LinCall {
  const QLinear* l;
  const float* A;
  int64_t M;
  int kind;
  const float* gate;
  float* Y;  // also the residual of the GATED / RESID kinds (in place)
};

namespace {

bool overlap(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b || !na || !nb) return false;
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + nb && pb < pa + na;
}

// The calls in order: one sdq_qlinear_group when no call's output overlaps
// another call's input or output (then the order cannot matter), else one
// call after the other.
void run_linears(const std::vector<LinCall>& calls, void* s) {
  bool independent = calls.size() <= SDQ_MAX_GROUP;
  for (size_t i = 0; independent && i < calls.size(); i++) {
    const LinCall& c = calls[i];
    const size_t yb = (size_t)(c.M * c.l->out_features()) * sizeof(float);
    for (size_t j = 0; j < calls.size(); j++) {
      if (i == j) continue;
      const LinCall& d = calls[j];
      const size_t ab = (size_t)(d.M * d.l->in_features()) * sizeof(float);
      const size_t db = (size_t)(d.M * d.l->out_features()) * sizeof(float);
      if (overlap(c.Y, yb, d.A, ab) || overlap(c.Y, yb, d.Y, db)) {
        independent = false;
        break;
      }
    }
  }
  auto epi = [](const LinCall& c) {
    const bool res = c.kind == SDQ_EPI_GATED || c.kind == SDQ_EPI_RESID;
    return sdq_epilogue{c.kind, 1, c.l->bias_device(), c.gate, res ? c.Y : nullptr};
  };
  if (!independent) {
    for (const LinCall& c : calls) c.l->forward_device(c.A, c.M, c.kind, c.gate, c.Y, c.Y, s);
    return;
  }
  std::vector<sdq_group_item> items;
  for (const LinCall& c : calls) items.push_back(sdq_group_item{c.l->handle(), c.A, c.M, epi(c), c.Y});
  check(sdq_qlinear_group(items.data(), (int)items.size(), s), "DitBlock linears");
}

sdq_group_item group_item(const LinCall& c) {
  const bool res = c.kind == SDQ_EPI_GATED || c.kind == SDQ_EPI_RESID;
  return sdq_group_item{c.l->handle(), c.A, c.M,
                        sdq_epilogue{c.kind, 1, c.l->bias_device(), c.gate, res ? c.Y : nullptr},
                        c.Y};
}

// `group` (independent), then `seq` in order, then the FFN when `ffn` is
// given, as one sdq_qlinear_stack: every input quantized by one launch. That
// needs every input in place before the first GEMM (no output overlaps an
// input) and `group` independent; otherwise the same calls run one by one.
void run_stack(const std::vector<LinCall>& group, const std::vector<LinCall>& seq,
               const sdq_ffn_item* ffn, int64_t D, int64_t F, void* s) {
  struct Buf {
    const void* p;
    size_t n;
  };
  std::vector<Buf> ins, outs;
  auto add = [&](const LinCall& c) {
    ins.push_back({c.A, (size_t)(c.M * c.l->in_features()) * sizeof(float)});
    outs.push_back({c.Y, (size_t)(c.M * c.l->out_features()) * sizeof(float)});
  };
  for (const LinCall& c : group) add(c);
  for (const LinCall& c : seq) add(c);
  if (ffn) {
    const size_t d = (size_t)D * sizeof(float), f = (size_t)F * sizeof(float);
    ins.push_back({ffn->h, (size_t)ffn->M * d});
    outs.push_back({ffn->hid, (size_t)ffn->M * f});
    outs.push_back({ffn->x, (size_t)ffn->M * d});
  }
  bool ok = group.size() + seq.size() <= SDQ_MAX_GROUP;
  for (const Buf& o : outs)
    for (const Buf& a : ins) ok = ok && !overlap(o.p, o.n, a.p, a.n);
  for (size_t i = 0; ok && i < group.size(); i++)
    for (size_t j = 0; j < group.size(); j++) {
      if (i == j) continue;
      const LinCall& c = group[i];
      const LinCall& d = group[j];
      ok = ok && !overlap(c.Y, (size_t)(c.M * c.l->out_features()) * sizeof(float), d.Y,
                          (size_t)(d.M * d.l->out_features()) * sizeof(float));
    }
  if (!ok) {
    run_linears(group, s);
    for (const LinCall& c : seq) run_linears({c}, s);
    if (ffn)
      check(sdq_ffn(ffn->fc1, ffn->b1, ffn->fc2, ffn->b2, ffn->h, ffn->M, ffn->gate,
                    ffn->gate_fma, ffn->hid, ffn->x, s),
            "DitBlock ffn");
    return;
  }
  std::vector<sdq_group_item> items;
  for (const LinCall& c : group) items.push_back(group_item(c));
  for (const LinCall& c : seq) items.push_back(group_item(c));
  check(sdq_qlinear_stack(items.data(), (int)items.size(), (int)group.size(), ffn, s),
        "DitBlock linear stack");
}

}  // namespace

// The FFN of the block as a stack entry, when it takes its normalized input
// from the caller (no norm + modulation folded into fc1's quantizer).
bool DitBlock::ffn_item(const sd_dit_block_io& io, sdq_ffn_item* f) const {
  if (io.shift_ffn && io.scale_ffn) return false;
  *f = sdq_ffn_item{fc1_.handle(), fc1_.bias_device(), fc2_.handle(), fc2_.bias_device(),
                    io.h_ffn,      io.M,               io.gate_ffn,   1,
                    io.hid,        io.x};
  return true;
}

// The Linears of the self and cross attention that read inputs the caller
// already has (ovi_dit.cpp:176-188, 229-254): q|k|v (unless the block
// normalizes x itself: then it runs first, from x), o into x, cross q, the
// text k|v, the fusion k|v.
void DitBlock::attn_linears(const sd_dit_block_io& io, std::vector<LinCall>& out) const {
  if (!(io.shift_sa && io.scale_sa))
    out.push_back({&qkv_, io.h_sa, io.M, SDQ_EPI_NONE, nullptr, io.qkv});
  out.push_back({&o_, io.att, io.M, SDQ_EPI_GATED, io.gate_sa, io.x});
  out.push_back({&cq_, io.xq, io.M, SDQ_EPI_NONE, nullptr, io.cq});
  if (io.Mc > 0) out.push_back({&ckv_, io.ctx, io.Mc, SDQ_EPI_NONE, nullptr, io.ckv});
  if (fusion_ && io.Mt > 0) out.push_back({&kvf_, io.tn, io.Mt, SDQ_EPI_NONE, nullptr, io.kvt});
}

void DitBlock::check_io(const sd_dit_block_io& io) const {
  need(io.M >= 0 && io.Mc >= 0 && io.Mt >= 0, "negative row count");
  need(io.x && io.gate_sa && io.gate_ffn, "x and gates are required");
}

void DitBlock::qkv_lnmod(const sd_dit_block_io& io, void* s) const {
  sdq_epilogue e{SDQ_EPI_NONE, 1, qkv_.bias_device(), nullptr, nullptr};
  check(sdq_qlinear_lnmod(qkv_.handle(), io.x, io.M, dim_, io.shift_sa, io.scale_sa, io.eps, &e,
                          io.qkv, s),
        "DitBlock q|k|v");
}

void DitBlock::ffn_linears(const sd_dit_block_io& io, void* s) const {
  // ffn: hid = gelu(fc1(h)); x += fc2(hid) * e[5]    (ovi_dit.cpp:214-222); one
  // call, so fc1's epilogue hands hid's row maxima to fc2's quantizer
  if (io.shift_ffn && io.scale_ffn)
    check(sdq_ffn_lnmod(fc1_.handle(), fc1_.bias_device(), fc2_.handle(), fc2_.bias_device(), io.x,
                        io.M, io.shift_ffn, io.scale_ffn, io.eps, io.gate_ffn, 1, io.hid, s),
          "DitBlock ffn");
  else
    check(sdq_ffn(fc1_.handle(), fc1_.bias_device(), fc2_.handle(), fc2_.bias_device(), io.h_ffn,
                  io.M, io.gate_ffn, 1, io.hid, io.x, s),
          "DitBlock ffn");
}

void DitBlock::forward_linears(const sd_dit_block_io& io, void* s) const {
  check_io(io);
  // self attention: q|k|v, then x += o(att) * e[2]   (ovi_dit.cpp:176-188, 205-212);
  // cross attention: q on tokens, k|v on the context, k_fusion|v_fusion on
  // the other branch (229-254). Independent given the inputs: one grouped
  // run when no output overlaps another Linear's input.
  // The whole stack from given inputs: every input quantized by one launch
  // (sdq_qlinear_stack), then the attention Linears grouped, x += o(xt) (251)
  // and the FFN in order.
  if (io.shift_sa && io.scale_sa) qkv_lnmod(io, s);
  std::vector<LinCall> calls;
  attn_linears(io, calls);
  sdq_ffn_item f;
  const bool fi = ffn_item(io, &f);
  run_stack(calls, {{&co_, io.xt, io.M, SDQ_EPI_RESID, nullptr, io.x}}, fi ? &f : nullptr, dim_,
            ffn_, s);
  if (!fi) ffn_linears(io, s);
}

namespace {

// A buffer one stream's work reads or writes (bytes).
struct Span {
  const void* p;
  size_t n;
  bool write;
};

// What a block's Linears read and write (forward_linears with io); `own`:
// q|k|v, o, cross q, cross o and the FFN; else the text k|v and fusion k|v
// (inputs the caller has from outside the branch: the context and the
// other branch's tokens).
std::vector<Span> linear_spans(const DitBlock& k, const sd_dit_block_io& io, bool own) {
  const size_t d = (size_t)k.dim() * sizeof(float), f = (size_t)k.ffn_dim() * sizeof(float);
  const size_t M = (size_t)io.M, Mc = (size_t)io.Mc, Mt = (size_t)io.Mt;
  if (!own)
    return {{io.ctx, Mc * d, false}, {io.ckv, 2 * Mc * d, true},
            {io.tn, Mt * d, false},  {io.kvt, 2 * Mt * d, true}};
  return {{io.h_sa, M * d, false},     {io.att, M * d, false},      {io.xq, M * d, false},
          {io.xt, M * d, false},       {io.h_ffn, M * d, false},    {io.gate_sa, d, false},
          {io.gate_ffn, d, false},     {io.shift_sa, d, false},     {io.scale_sa, d, false},
          {io.shift_ffn, d, false},    {io.scale_ffn, d, false},    {io.qkv, 3 * M * d, true},
          {io.cq, M * d, true},        {io.hid, M * f, true},       {io.x, M * d, true}};
}

// Whether two sets of work may run at the same time: neither writes what
// the other reads or writes.
bool disjoint(const std::vector<Span>& u, const std::vector<Span>& v) {
  for (const Span& a : u)
    for (const Span& b : v)
      if ((a.write || b.write) && overlap(a.p, a.n, b.p, b.n)) return false;
  return true;
}

}  // namespace

void forward_linears_pair(const DitBlock& a, const sd_dit_block_io& ia, const DitBlock& b,
                          const sd_dit_block_io& ib, void* s, void* s2) {
  a.check_io(ia);
  b.check_io(ib);
  if (s2 && s2 != s) {
    // Two streams: a's own Linears on s; b's, and a's text k|v and fusion
    // k|v (which need nothing from a's branch), on s2 (the streams' loads
    // balance: a is the longer branch). Only when neither side touches what
    // the other writes.
    std::vector<Span> on_s = linear_spans(a, ia, true), on_s2 = linear_spans(a, ia, false);
    for (const Span& x : linear_spans(b, ib, true)) on_s2.push_back(x);
    for (const Span& x : linear_spans(b, ib, false)) on_s2.push_back(x);
    if (disjoint(on_s, on_s2)) {
      check(sdq_stream_wait(s2, s), "pair fork");
      if (ia.shift_sa && ia.scale_sa) a.qkv_lnmod(ia, s);
      if (ib.shift_sa && ib.scale_sa) b.qkv_lnmod(ib, s2);
      std::vector<LinCall> ca, cb, ctx;
      a.attn_linears(ia, ca);
      // a's text k|v and fusion k|v move to s2 (they read ctx / tn)
      for (auto it = ca.begin(); it != ca.end();) {
        if (it->l == &a.ckv_ || it->l == &a.kvf_) {
          ctx.push_back(*it);
          it = ca.erase(it);
        } else {
          ++it;
        }
      }
      b.attn_linears(ib, cb);
      for (const LinCall& c : ctx) cb.push_back(c);
      sdq_ffn_item fa, fb;
      const bool ha = a.ffn_item(ia, &fa), hb = b.ffn_item(ib, &fb);
      run_stack(ca, {{&a.co_, ia.xt, ia.M, SDQ_EPI_RESID, nullptr, ia.x}}, ha ? &fa : nullptr,
                a.dim(), a.ffn_dim(), s);
      run_stack(cb, {{&b.co_, ib.xt, ib.M, SDQ_EPI_RESID, nullptr, ib.x}}, hb ? &fb : nullptr,
                b.dim(), b.ffn_dim(), s2);
      if (!ha) a.ffn_linears(ia, s);
      if (!hb) b.ffn_linears(ib, s2);
      check(sdq_stream_wait(s, s2), "pair join");
      return;
    }
  }
  if (ia.shift_sa && ia.scale_sa) a.qkv_lnmod(ia, s);
  if (ib.shift_sa && ib.scale_sa) b.qkv_lnmod(ib, s);
  std::vector<LinCall> calls;
  a.attn_linears(ia, calls);
  b.attn_linears(ib, calls);
  run_linears(calls, s);
  run_linears({{&a.co_, ia.xt, ia.M, SDQ_EPI_RESID, nullptr, ia.x},
               {&b.co_, ib.xt, ib.M, SDQ_EPI_RESID, nullptr, ib.x}},
              s);
  a.ffn_linears(ia, s);
  b.ffn_linears(ib, s);
}

void DitBlock::set_norms(const sd_dit_norms& n) {
  const float* v[kNorms] = {n.sa_nq, n.sa_nk, n.ca_nq, n.ca_nk, n.ln3_w,
                            n.ln3_b, n.nk_fusion, n.pnf_w, n.pnf_b};
  need(v[SA_NQ] && v[SA_NK] && v[CA_NQ] && v[CA_NK], "attention norm weights are required");
  if (fusion_)
    need(v[NK_F] && v[PNF_W] && v[PNF_B], "fusion blocks need norm_k_fusion and pre_attn_norm_fusion");
  else
    need(v[LN3_W] && v[LN3_B], "norm3 weight and bias are required");
  std::vector<float> h((size_t)kNorms * dim_, 0.f);
  for (int i = 0; i < kNorms; i++)
    if (v[i]) std::copy(v[i], v[i] + dim_, h.begin() + (size_t)i * dim_);
  DeviceFloats d(h.size());
  check(sdq_memcpy(d.get(), h.data(), h.size() * sizeof(float), SDQ_H2D, nullptr), "norm upload");
  check(sdq_stream_sync(nullptr), "norm upload");
  norms_ = std::move(d);
}

void DitBlock::set_modulation(const float* mod) {
  need(mod != nullptr, "modulation bias is required");
  DeviceFloats d((size_t)6 * dim_);
  check(sdq_memcpy(d.get(), mod, (size_t)6 * dim_ * sizeof(float), SDQ_H2D, nullptr),
        "modulation upload");
  check(sdq_stream_sync(nullptr), "modulation upload");
  mod_ = std::move(d);
}

// e = t6 + mod, value by value (the reference adds the block's bias into a
// copy of the time rows, ovi_dit.cpp:716-723): a copy, then x += y.
void DitBlock::modulation_rows(const float* t6, float* e, void* s) const {
  need(static_cast<bool>(mod_), "modulation bias not set (set_modulation)");
  need(t6 && e, "t6 and e are required");
  const size_t n = (size_t)6 * dim_;
  if (e != t6) check(sdq_memcpy(e, t6, n * sizeof(float), SDQ_D2D, s), "modulation rows");
  check(sdq_add(e, mod_.get(), (int64_t)n, s), "modulation rows");
}

namespace {

// Workspace carve-up (floats, each region 256-byte aligned): a [M,3dim]
// (self: q|k|v; cross: q, text attention output, norm3 output or target
// attention output), att [M,dim], ckv [Mc,2dim], tn [Mt,dim], kvt [Mt,2dim],
// hid [M,ffn].
struct Carve {
  int64_t a, att, ckv, tn, kvt, hid, total;
};

int64_t up64(int64_t n) { return (n + 63) / 64 * 64; }

Carve carve(int64_t M, int64_t Mc, int64_t Mt, int64_t C, int64_t F, bool fusion) {
  Carve c{};
  int64_t o = 0;
  c.a = o, o += up64(3 * M * C);
  c.att = o, o += up64(M * C);
  c.ckv = o, o += up64(2 * Mc * C);
  c.tn = o, o += fusion ? up64(Mt * C) : 0;
  c.kvt = o, o += fusion ? up64(2 * Mt * C) : 0;
  c.hid = o, o += up64(M * F);
  c.total = o;
  return c;
}

}  // namespace

size_t DitBlock::workspace_bytes(int64_t M, int64_t Mc, int64_t Mt) const {
  return (size_t)carve(M, Mc, Mt, dim_, ffn_, fusion_).total * sizeof(float);
}

// block_self_fwd (ovi_dit.cpp:205-212) with self_attn_fwd (176-188):
// q|k|v = mlin(mod_rows(layernorm(x), e0, e1)); rmsnorm + RoPE on q and k;
// x += o(sdpa(q, k, v)) * e2.
void DitBlock::self_phase(const sd_dit_block_step& st, int batch, float* ws, void* s) const {
  // `batch` sequences stacked along the rows: every step is per row except
  // the attention, which stays inside each sequence
  const int64_t C = dim_, M = st.M, BM = batch * M;
  const Carve c = carve(BM, batch * st.Mc, batch * st.Mt, C, ffn_, fusion_);
  float* qkv = ws + c.a;
  float* att = ws + c.att;
  sdq_epilogue epi{SDQ_EPI_NONE, 1, qkv_.bias_device(), nullptr, nullptr};
  check(sdq_qlinear_lnmod(qkv_.handle(), st.x, BM, C, st.e, st.e + C, st.eps, &epi, qkv, s),
        "self q|k|v");
  // q and k norms (+ RoPE) in one launch: two independent serial row-sum sets
  const int nr = st.cs ? st.nr : 0;
  const sdq_rms_seg qk[2] = {{qkv, BM, 3 * C, norm(SA_NQ), st.cs, nr},
                             {qkv + C, BM, 3 * C, norm(SA_NK), st.cs, nr}};
  check(sdq_rmsnorm_rope_batch(qk, 2, C, st.heads, st.eps, s), "self rmsnorm+rope q, k");
  check(sdq_sdpa_batched(qkv, 3 * C, qkv + C, 3 * C, qkv + 2 * C, 3 * C, att, C, M, M, st.heads,
                         (int)(C / st.heads), batch, s),
        "self sdpa");
  o_.forward_device(att, BM, SDQ_EPI_GATED, st.e + 2 * C, st.x, st.x, s);
}

// Non-fusion blocks (block_vanilla_fwd, ovi_dit.cpp:259-268 with
// cross_text_fwd 191-201): x += o(sdpa(rmsnorm(q(norm3(x))), rmsnorm(k(ctx)),
// v(ctx))). Fusion blocks (fusion_cross_ffn, 229-256): q on x itself; the
// text attention uses q unrotated, then q is rotated with this branch's
// table for the attention on the target's k_fusion (rmsnorm + the target's
// table) and v_fusion of layernorm(target; pre_attn_norm_fusion); x +=
// o(text + target attention). Then ffn_fwd (214-222).
void DitBlock::cross_ffn_phase(const sd_dit_block_step& st, int batch, float* ws, void* s) const {
  const int64_t C = dim_, M = st.M, Mc = st.Mc, Mt = st.Mt;
  const int64_t BM = batch * M, BMc = batch * Mc, BMt = batch * Mt;
  const int hd = (int)(C / st.heads);
  const Carve c = carve(BM, BMc, BMt, C, ffn_, fusion_);
  float* cq = ws + c.a;
  float* xt = ws + c.a + BM * C;
  float* aux = ws + c.a + 2 * BM * C;  // norm3 output, then the target attention
  float* ckv = ws + c.ckv;
  const float* qin = st.x;
  if (!fusion_) {
    check(sdq_layernorm(st.x, BM, C, norm(LN3_W), norm(LN3_B), st.eps, aux, s), "norm3");
    qin = aux;
  }
  // cross q, the text k|v and the fusion k|v (on the layernormed target)
  // read inputs that are ready here: one grouped run
  float* kvt = ws + c.kvt;
  std::vector<LinCall> calls{{&cq_, qin, BM, SDQ_EPI_NONE, nullptr, cq},
                             {&ckv_, st.ctx, BMc, SDQ_EPI_NONE, nullptr, ckv}};
  if (fusion_) {
    float* tn = ws + c.tn;
    check(sdq_layernorm(st.target, BMt, C, norm(PNF_W), norm(PNF_B), st.eps, tn, s),
          "pre_attn_norm_fusion");
    calls.push_back({&kvf_, tn, BMt, SDQ_EPI_NONE, nullptr, kvt});
  }
  run_linears(calls, s);
  // rmsnorm of cross q and context k (no rotation); fusion: rmsnorm_k_fusion
  // + the target's rotation of k_fusion. Independent row sets, one launch.
  const sdq_rms_seg nk[3] = {{cq, BM, C, norm(CA_NQ), nullptr, 0},
                             {ckv, BMc, 2 * C, norm(CA_NK), nullptr, 0},
                             {kvt, BMt, 2 * C, norm(NK_F), st.cs_tgt, st.cs_tgt ? st.nr_tgt : 0}};
  check(sdq_rmsnorm_rope_batch(nk, fusion_ ? 3 : 2, C, st.heads, st.eps, s), "cross norms");
  check(sdq_sdpa_batched(cq, C, ckv, 2 * C, ckv + C, 2 * C, xt, C, M, Mc, st.heads, hd, batch, s),
        "text sdpa");
  if (fusion_) {
    if (st.cs)
      check(sdq_rmsnorm_rope(cq, BM, C, C, nullptr, st.eps, st.heads, st.cs, st.nr, s), "rope q");
    check(sdq_sdpa_batched(cq, C, kvt, 2 * C, kvt + C, 2 * C, aux, C, M, Mt, st.heads, hd, batch,
                           s),
          "target sdpa");
    check(sdq_add(xt, aux, BM * C, s), "text + target");
  }
  co_.forward_device(xt, BM, SDQ_EPI_RESID, nullptr, st.x, st.x, s);
  const float* e = st.e;
  check(sdq_ffn_lnmod(fc1_.handle(), fc1_.bias_device(), fc2_.handle(), fc2_.bias_device(), st.x,
                      BM, e + 3 * C, e + 4 * C, st.eps, e + 5 * C, 1, ws + c.hid, s),
        "ffn");
}

void DitBlock::forward_step(const sd_dit_block_step& st, int phases, void* s, int batch) const {
  need(norms_.get() != nullptr, "norm weights not set (set_norms)");
  need(phases >= 1 && phases <= 3, "phases must be SD_DIT_SELF, SD_DIT_CROSS_FFN or both");
  need(batch >= 1 && batch <= 64, "batch must be 1..64");
  need(st.M >= 0 && st.Mc > 0 && st.Mt >= 0, "row counts (M >= 0, Mc > 0)");
  need(st.heads > 0 && dim_ % st.heads == 0 && dim_ / st.heads == 128, "head_dim must be 128");
  need(st.x && st.e, "x and e are required");
  need(st.ws && st.ws_bytes >= workspace_bytes(batch * st.M, batch * st.Mc, batch * st.Mt),
       "workspace too small");
  if (st.M == 0) return;
  const int64_t hd = dim_ / st.heads;
  need(!st.cs || (st.nr > 0 && st.nr <= hd / 2), "rope table pairs out of range");
  float* ws = static_cast<float*>(st.ws);
  if (phases & SD_DIT_SELF) self_phase(st, batch, ws, s);
  if (phases & SD_DIT_CROSS_FFN) {
    need(st.ctx, "ctx is required");
    if (fusion_) {
      need(st.target && st.Mt > 0, "fusion blocks need the target tokens");
      need(!st.cs_tgt || (st.nr_tgt > 0 && st.nr_tgt <= hd / 2), "target rope pairs out of range");
    }
    cross_ffn_phase(st, batch, ws, s);
  }
}

double DitBlock::step_ops(int64_t M, int64_t Mc, int64_t Mt) const {
  const double d = (double)dim_;
  double o = ops(M, Mc, fusion_ ? Mt : 0);
  o += 4.0 * M * M * d + 4.0 * M * Mc * d;
  if (fusion_) o += 4.0 * M * Mt * d;
  return o;
}

double DitBlock::ops(int64_t M, int64_t Mc, int64_t Mt) const {
  const double d = (double)dim_, f = (double)ffn_;
  double o = 2.0 * M * d * (3 * d) + 2.0 * M * d * d * 3 + 2.0 * Mc * d * (2 * d) +
             2.0 * M * d * f * 2;
  if (fusion_) o += 2.0 * Mt * d * (2 * d);
  return o;
}

namespace {

// The block's Linears as lin() checks them (ovi_dit.cpp:397-415, 505-530).
void block_parts(const std::unordered_map<std::string, Tensor>& pack, const std::string& prefix,
                 int layer, int64_t dim, int64_t ffn_dim, bool fusion, LinearPart* l) {
  const std::string B = prefix + "blocks." + std::to_string(layer) + ".";
  l[DitBlock::Q] = linear_part_from_pack(pack, B + "self_attn.q", dim, dim);
  l[DitBlock::K] = linear_part_from_pack(pack, B + "self_attn.k", dim, dim);
  l[DitBlock::V] = linear_part_from_pack(pack, B + "self_attn.v", dim, dim);
  l[DitBlock::O] = linear_part_from_pack(pack, B + "self_attn.o", dim, dim);
  l[DitBlock::CQ] = linear_part_from_pack(pack, B + "cross_attn.q", dim, dim);
  l[DitBlock::CK] = linear_part_from_pack(pack, B + "cross_attn.k", dim, dim);
  l[DitBlock::CV] = linear_part_from_pack(pack, B + "cross_attn.v", dim, dim);
  l[DitBlock::CO] = linear_part_from_pack(pack, B + "cross_attn.o", dim, dim);
  if (fusion) {
    l[DitBlock::KF] = linear_part_from_pack(pack, B + "cross_attn.k_fusion", dim, dim);
    l[DitBlock::VF] = linear_part_from_pack(pack, B + "cross_attn.v_fusion", dim, dim);
  }
  l[DitBlock::FC1] = linear_part_from_pack(pack, B + "ffn.0", dim, ffn_dim);
  l[DitBlock::FC2] = linear_part_from_pack(pack, B + "ffn.2", ffn_dim, dim);
}

}  // namespace

namespace {

// The block's small F32 tensors (vec() and the modulation check of
// load_impl, ovi_dit.cpp:417-422, 509-537), from any source of F32 values:
// get(name, &dims) returns the values and shape, or throws "missing tensor".
struct BlockVectors {
  std::vector<float> v[9];  // sd_dit_norms order
  std::vector<float> mod;   // [6, dim]
};

template <class Get>
BlockVectors block_vectors(Get get, const std::string& prefix, int layer, int64_t dim,
                           bool fusion) {
  const std::string B = prefix + "blocks." + std::to_string(layer) + ".";
  BlockVectors out;
  auto vec = [&](int slot, const std::string& n) {
    std::vector<int64_t> dims;
    std::vector<float> v = get(n, dims);
    if (dims.size() != 1 || dims[0] != dim) throw std::runtime_error("ovi_dit: bad shape for " + n);
    out.v[slot] = std::move(v);
  };
  vec(0, B + "self_attn.norm_q.weight");
  vec(1, B + "self_attn.norm_k.weight");
  vec(2, B + "cross_attn.norm_q.weight");
  vec(3, B + "cross_attn.norm_k.weight");
  vec(4, B + "norm3.weight");
  vec(5, B + "norm3.bias");
  std::vector<int64_t> md;
  out.mod = get(B + "modulation.modulation", md);
  if (md.size() != 3 || md[0] != 1 || md[1] != 6 || md[2] != dim)
    throw std::runtime_error("ovi_dit: bad modulation " + B);
  if (fusion) {
    vec(6, B + "cross_attn.norm_k_fusion.weight");
    vec(7, B + "cross_attn.pre_attn_norm_fusion.weight");
    vec(8, B + "cross_attn.pre_attn_norm_fusion.bias");
  }
  return out;
}

void apply_vectors(DitBlock& b, const BlockVectors& bv) {
  auto p = [&](int i) { return bv.v[i].empty() ? nullptr : bv.v[i].data(); };
  const sd_dit_norms n{p(0), p(1), p(2), p(3), p(4), p(5), p(6), p(7), p(8)};
  b.set_norms(n);
  b.set_modulation(bv.mod.data());
}

// F32 values of a load_sdcpp view (the reference's vec() would dequantize an
// int8 entry; packs never quantize these small tensors).
std::vector<float> view_values(const std::unordered_map<std::string, Tensor>& pack,
                               const std::string& name, std::vector<int64_t>& dims) {
  auto it = pack.find(name);
  if (it == pack.end() || !it->second.data) throw std::runtime_error("ovi_dit: missing tensor " + name);
  const Tensor& t = it->second;
  if (t.dtype != DType::F32)
    throw std::runtime_error("ovi_dit: " + name + " is not an F32 pack entry");
  dims = t.shape;
  const float* f = t.ptr<float>();
  return std::vector<float>(f, f + t.numel());
}

}  // namespace

DitBlock dit_block_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                             const std::string& prefix, int layer, int64_t dim, int64_t ffn_dim,
                             bool fusion) {
  LinearPart l[DitBlock::kCount];
  block_parts(pack, prefix, layer, dim, ffn_dim, fusion, l);
  const BlockVectors bv = block_vectors(
      [&](const std::string& n, std::vector<int64_t>& d) { return view_values(pack, n, d); },
      prefix, layer, dim, fusion);
  DitBlock b(l, fusion, false);
  apply_vectors(b, bv);
  return b;
}

std::vector<DitBlock> dit_blocks_from_pack(const std::unordered_map<std::string, Tensor>& pack,
                                           const std::string& prefix,
                                           const std::vector<int>& layers, int64_t dim,
                                           int64_t ffn_dim, bool fusion) {
  std::vector<std::array<LinearPart, DitBlock::kCount>> parts(layers.size());
  std::vector<BlockVectors> vecs;
  for (size_t i = 0; i < layers.size(); i++) {
    block_parts(pack, prefix, layers[i], dim, ffn_dim, fusion, parts[i].data());
    vecs.push_back(block_vectors(
        [&](const std::string& n, std::vector<int64_t>& d) { return view_values(pack, n, d); },
        prefix, layers[i], dim, fusion));
  }
  std::vector<DitBlock> blocks = DitBlock::create_many(parts, fusion);
  for (size_t i = 0; i < blocks.size(); i++) apply_vectors(blocks[i], vecs[i]);
  return blocks;
}

namespace {

// lin() on the pack index (ovi_dit.cpp:397-415): the same names, checks and
// messages as linear_part_from_pack on load_sdcpp's views.
FilePart file_part(const PackIndex& ix, const std::string& base, int64_t in, int64_t out) {
  const std::string wn = base + ".weight";
  const PackEntry* w = ix.find(wn);
  if (!w) throw std::runtime_error("ovi_dit: missing tensor " + wn);
  if (w->dims.size() != 2 || w->dims[0] != out || w->dims[1] != in)
    throw std::runtime_error("ovi_dit: bad shape for " + wn);
  if (w->kind != PackEntry::kInt8Rows)
    throw std::runtime_error("ovi_dit: " + wn + " is not an int8 pack entry");
  bool from_int8 = false;
  const PackEntry* sc = ix.f32_view(wn + ".scale", &from_int8);
  if (!sc) throw std::runtime_error("ovi_dit: missing tensor " + wn + ".scale");
  // where the view's floats start, checked as lin() checks its pointers
  const uint64_t sc_at = from_int8 ? sc->scale : sc->data;
  if (sc_at != w->data + (uint64_t)w->numel)
    throw std::runtime_error("ovi_dit: scale not packed after i8 for " + base);
  bool bias_scale = false;
  const PackEntry* b = ix.f32_view(base + ".bias", &bias_scale);
  if (!b) throw std::runtime_error("ovi_dit: missing tensor " + base + ".bias");
  const int64_t bn = bias_scale ? b->rows : b->numel;
  if ((!bias_scale && b->dims.size() != 1) || bn != out)
    throw std::runtime_error("ovi_dit: bad shape for " + base + ".bias");
  FilePart p;
  p.q_off = w->data;
  p.scale_off = w->scale;
  p.bias = ix.read_f32(*b, bias_scale);
  p.out = out;
  p.in = in;
  return p;
}

std::vector<float> index_values(const PackIndex& ix, const std::string& name,
                                std::vector<int64_t>& dims) {
  bool is_scale = false;
  const PackEntry* e = ix.f32_view(name, &is_scale);
  if (!e) {
    if (ix.find(name)) throw std::runtime_error("ovi_dit: " + name + " is not an F32 pack entry");
    throw std::runtime_error("ovi_dit: missing tensor " + name);
  }
  dims = is_scale ? std::vector<int64_t>{e->rows} : e->dims;
  return ix.read_f32(*e, is_scale);
}

}  // namespace

std::vector<DitBlock> dit_blocks_from_pack_file(const std::string& path, const std::string& prefix,
                                                const std::vector<int>& layers, int64_t dim,
                                                int64_t ffn_dim, bool fusion) {
  const PackIndex ix = PackIndex::read(path);
  std::vector<std::vector<FilePart>> sets;
  std::vector<BlockVectors> vecs;
  for (int layer : layers) {
    const std::string B = prefix + "blocks." + std::to_string(layer) + ".";
    auto fp = [&](const char* n, int64_t in, int64_t out) { return file_part(ix, B + n, in, out); };
    FilePart q = fp("self_attn.q", dim, dim), k = fp("self_attn.k", dim, dim),
             v = fp("self_attn.v", dim, dim), o = fp("self_attn.o", dim, dim);
    FilePart cq = fp("cross_attn.q", dim, dim), ck = fp("cross_attn.k", dim, dim),
             cv = fp("cross_attn.v", dim, dim), co = fp("cross_attn.o", dim, dim);
    FilePart fc1 = fp("ffn.0", dim, ffn_dim), fc2 = fp("ffn.2", ffn_dim, dim);
    sets.push_back({std::move(q), std::move(k), std::move(v)});
    sets.push_back({std::move(o)});
    sets.push_back({std::move(cq)});
    sets.push_back({std::move(ck), std::move(cv)});
    if (fusion)
      sets.push_back({fp("cross_attn.k_fusion", dim, dim), fp("cross_attn.v_fusion", dim, dim)});
    sets.push_back({std::move(co)});
    sets.push_back({std::move(fc1)});
    sets.push_back({std::move(fc2)});
    vecs.push_back(block_vectors(
        [&](const std::string& n, std::vector<int64_t>& d) { return index_values(ix, n, d); },
        prefix, layer, dim, fusion));
  }
  std::vector<QLinear> q = QLinear::upload_many_file(path, sets);
  std::vector<DitBlock> out;
  out.reserve(layers.size());
  size_t j = 0;
  for (size_t b = 0; b < layers.size(); b++) {
    DitBlock d;
    d.fusion_ = fusion;
    d.dim_ = dim;
    d.ffn_ = ffn_dim;
    d.qkv_ = std::move(q[j++]);
    d.o_ = std::move(q[j++]);
    d.cq_ = std::move(q[j++]);
    d.ckv_ = std::move(q[j++]);
    if (fusion) d.kvf_ = std::move(q[j++]);
    d.co_ = std::move(q[j++]);
    d.fc1_ = std::move(q[j++]);
    d.fc2_ = std::move(q[j++]);
    apply_vectors(d, vecs[b]);
    out.push_back(std::move(d));
  }
  return out;
}

}  // namespace gpu
}  // namespace sd

// ---- C shim (tests, bench, non-C++ callers) ----
struct sd_dit_block {
  sd::gpu::DitBlock blk;
};

namespace {
thread_local std::string t_dit_err;

template <class F>
int guarded(F&& f) {
  try {
    f();
    return SDQ_OK;
  } catch (const std::exception& e) {
    t_dit_err = e.what();
    return SDQ_ERR_INVALID;
  }
}
}  // namespace

extern "C" {

const char* sd_dit_last_error(void) { return t_dit_err.c_str(); }

int sd_dit_block_create(const sd_linear* lin, int fusion, int on_device, sd_dit_block** out) {
  if (!lin || !out) {
    t_dit_err = "sd_dit_block_create: null argument";
    return SDQ_ERR_INVALID;
  }
  *out = nullptr;
  return guarded([&] {
    sd::gpu::LinearPart l[sd::gpu::DitBlock::kCount];
    for (int i = 0; i < sd::gpu::DitBlock::kCount; i++) {
      if (!fusion && (i == sd::gpu::DitBlock::KF || i == sd::gpu::DitBlock::VF)) continue;
      l[i].w = lin[i].w;
      l[i].scale = lin[i].scale;
      l[i].bias = lin[i].bias;
      l[i].out = lin[i].out;
      l[i].in = lin[i].in;
    }
    *out = new sd_dit_block{sd::gpu::DitBlock(l, fusion != 0, on_device != 0)};
  });
}

int sd_dit_block_create_many(const sd_linear* lin, int nblocks, int fusion, sd_dit_block** out) {
  if (!lin || !out || nblocks < 0) {
    t_dit_err = "sd_dit_block_create_many: null argument or negative count";
    return SDQ_ERR_INVALID;
  }
  for (int b = 0; b < nblocks; b++) out[b] = nullptr;
  return guarded([&] {
    using sd::gpu::DitBlock;
    std::vector<std::array<sd::gpu::LinearPart, DitBlock::kCount>> parts(nblocks);
    for (int b = 0; b < nblocks; b++)
      for (int i = 0; i < DitBlock::kCount; i++) {
        if (!fusion && (i == DitBlock::KF || i == DitBlock::VF)) continue;
        const sd_linear& s = lin[b * DitBlock::kCount + i];
        parts[b][i] = sd::gpu::LinearPart{s.w, s.scale, s.bias, s.out, s.in};
      }
    std::vector<DitBlock> blocks = DitBlock::create_many(parts, fusion != 0);
    for (int b = 0; b < nblocks; b++) out[b] = new sd_dit_block{std::move(blocks[b])};
  });
}

int sd_dit_block_forward(const sd_dit_block* b, const sd_dit_block_io* io, void* stream) {
  if (!b || !io) {
    t_dit_err = "sd_dit_block_forward: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { b->blk.forward_linears(*io, stream); });
}

int sd_dit_block_forward_pair(const sd_dit_block* a, const sd_dit_block_io* ia,
                              const sd_dit_block* b, const sd_dit_block_io* ib, void* stream) {
  if (!a || !ia || !b || !ib) {
    t_dit_err = "sd_dit_block_forward_pair: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { sd::gpu::forward_linears_pair(a->blk, *ia, b->blk, *ib, stream); });
}

int sd_dit_block_forward_pair2(const sd_dit_block* a, const sd_dit_block_io* ia,
                               const sd_dit_block* b, const sd_dit_block_io* ib, void* stream,
                               void* stream2) {
  if (!a || !ia || !b || !ib) {
    t_dit_err = "sd_dit_block_forward_pair2: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded(
      [&] { sd::gpu::forward_linears_pair(a->blk, *ia, b->blk, *ib, stream, stream2); });
}

int sd_dit_block_free(sd_dit_block* b) {
  delete b;
  return SDQ_OK;
}

double sd_dit_block_ops(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt) {
  return b ? b->blk.ops(M, Mc, Mt) : 0.0;
}

int sd_dit_block_set_norms(sd_dit_block* b, const sd_dit_norms* n) {
  if (!b || !n) {
    t_dit_err = "sd_dit_block_set_norms: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { b->blk.set_norms(*n); });
}

int sd_dit_block_set_modulation(sd_dit_block* b, const float* mod) {
  if (!b || !mod) {
    t_dit_err = "sd_dit_block_set_modulation: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { b->blk.set_modulation(mod); });
}

int sd_dit_block_modulation(const sd_dit_block* b, const float* t6, float* e, void* stream) {
  if (!b) {
    t_dit_err = "sd_dit_block_modulation: null block";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { b->blk.modulation_rows(t6, e, stream); });
}

int sd_dit_blocks_from_pack(const char* path, const char* prefix, const int* layers, int n,
                            int64_t dim, int64_t ffn_dim, int fusion, int file_reads,
                            sd_dit_block** out) {
  if (!path || !prefix || !out || n < 0 || (n > 0 && !layers)) {
    t_dit_err = "sd_dit_blocks_from_pack: null argument or negative count";
    return SDQ_ERR_INVALID;
  }
  for (int i = 0; i < n; i++) out[i] = nullptr;
  return guarded([&] {
    const std::vector<int> ls(layers, layers + n);
    std::vector<sd::gpu::DitBlock> blocks;
    if (file_reads) {
      blocks = sd::gpu::dit_blocks_from_pack_file(path, prefix, ls, dim, ffn_dim, fusion != 0);
    } else {
      std::shared_ptr<void> owner;
      const auto pack = sd::load_sdcpp(path, owner);
      blocks = sd::gpu::dit_blocks_from_pack(pack, prefix, ls, dim, ffn_dim, fusion != 0);
    }
    for (int i = 0; i < n; i++) out[i] = new sd_dit_block{std::move(blocks[i])};
  });
}

size_t sd_dit_block_workspace_bytes(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt) {
  return b && M >= 0 && Mc >= 0 && Mt >= 0 ? b->blk.workspace_bytes(M, Mc, Mt) : 0;
}

int sd_dit_block_step_forward(const sd_dit_block* b, const sd_dit_block_step* st, int phases,
                              void* stream) {
  return sd_dit_block_step_forward_batched(b, st, 1, phases, stream);
}

int sd_dit_block_step_forward_batched(const sd_dit_block* b, const sd_dit_block_step* st,
                                      int batch, int phases, void* stream) {
  if (!b || !st) {
    t_dit_err = "sd_dit_block_step_forward: null argument";
    return SDQ_ERR_INVALID;
  }
  return guarded([&] { b->blk.forward_step(*st, phases, stream, batch); });
}

double sd_dit_block_step_ops(const sd_dit_block* b, int64_t M, int64_t Mc, int64_t Mt) {
  return b ? b->blk.step_ops(M, Mc, Mt) : 0.0;
}

}  // extern "C"
