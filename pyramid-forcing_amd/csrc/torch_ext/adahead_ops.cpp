// torch binding of the pyramid KV-cache path: TORCH_LIBRARY(adahead) with
// the reference's op schemas and the PyramidKVCacheManager custom class
// (reference: pyramidkv/csrc/scatter_copy_bind.cpp:763-982,
// pyramidkv_manager.{h,cc}).  Host C++ only: every op validates its
// arguments like the reference, then calls the C ABI of
// libpyramidkv_hip.so (include/pyramidkv_hip.h) with raw device pointers and
// the current HIP stream.  Ops added by this build (ragged_attention,
// rope_apply, cache_update, mega_merge_accum_weighted and the dit_* row
// operations of the end-to-end rollout's model) are registered in
// the same namespace.

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <cstring>
#include <string>
#include <tuple>
#include <vector>

#include "pyramidkv_hip.h"

namespace adahead {

using at::Tensor;

static void pkv_check(int rc, const char *what) {
  if (rc == PKV_OK) return;
  const char *msg = pkv_last_error();
  TORCH_CHECK(false, what, ": ", msg ? msg : "(no message)");
}

static pkv_stream_t stream_for(const Tensor &t) {
  return reinterpret_cast<pkv_stream_t>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

template <typename T>
static T *ptr_or_null(const Tensor &t) {
  return (t.defined() && t.numel() > 0) ? reinterpret_cast<T *>(t.data_ptr()) : nullptr;
}

static void check_i32(const Tensor &t, const char *name) {
  TORCH_CHECK(t.scalar_type() == at::kInt, name, " must be int32");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

constexpr int64_t kMaxMergeBlocks = 6, kMaxMergeActive = 2, kMaxMergeTokens = 420;

// `t` is a contiguous tensor of `dtype` and exactly `shape` on `dev`.
static void expect_tensor(const Tensor &t, at::ScalarType dtype, at::IntArrayRef shape, const c10::Device &dev,
                          const char *op, const char *name) {
  TORCH_CHECK(t.defined() && t.device() == dev, op, ": ", name, " must be on ", dev, " (got ",
              t.defined() ? t.device().str() : std::string("undefined"), ")");
  TORCH_CHECK(t.scalar_type() == dtype, op, ": ", name, " must be ", dtype, " (got ", t.scalar_type(), ")");
  TORCH_CHECK(t.sizes() == shape, op, ": ", name, " must be ", shape, " (got ", t.sizes(), ")");
  TORCH_CHECK(t.is_contiguous(), op, ": ", name, " must be contiguous");
}

// A descriptor array the kernels write: contiguous int32 on `dev` with at
// least n entries.
static void expect_desc(const Tensor &t, int64_t n, const c10::Device &dev, const char *op) {
  TORCH_CHECK(t.device() == dev && t.scalar_type() == at::kInt && t.is_contiguous() && t.numel() >= n, op,
              ": descriptor tensors must be contiguous int32 on ", dev, " with at least ", n, " entries (got ",
              t.scalar_type(), " ", t.numel(), " on ", t.device(), ")");
}

// One layer's Veil merge tensors, with the extents every merge kernel
// indexes: accumulators [H, MMA, MTPA, D] fp32, their positions
// [H, MMA, MTPA, 3] int64, group ids [H, MMA, FSEQ] int32, tokens per group
// [H, MMA, MTPA] fp32, group counts [H, MMA] int32 (weight sums [H, MMA] fp32
// when given); the merge pools [H, MMB, MTPA, D] bf16, their positions
// [H, MMB, MTPA, 3] int64 and token counts [H, MMB] int32.  MMA and MTPA are
// read from acc_k, MMB from mk.
static void expect_merge_layer(const char *op, const c10::Device &dev, int64_t H, int64_t FSEQ, int64_t D,
                               const Tensor &acc_k, const Tensor &acc_v, const Tensor &acc_pos, const Tensor &acc_gid,
                               const Tensor &acc_tpg, const Tensor &acc_ng, const Tensor *acc_wsum, const Tensor &mk,
                               const Tensor &mv, const Tensor &mpos, const Tensor &mtc) {
  TORCH_CHECK(acc_k.dim() == 4 && mk.dim() == 4, op, ": accum_sum_k must be [H, MMA, MTPA, D] and merge_k_pool "
              "[H, MMB, MTPA, D]");
  const int64_t MMA = acc_k.size(1), MTPA = acc_k.size(2), MMB = mk.size(1);
  expect_tensor(acc_k, at::kFloat, {H, MMA, MTPA, D}, dev, op, "accum_sum_k");
  expect_tensor(acc_v, at::kFloat, {H, MMA, MTPA, D}, dev, op, "accum_sum_v");
  expect_tensor(acc_pos, at::kLong, {H, MMA, MTPA, 3}, dev, op, "accum_pos");
  expect_tensor(acc_gid, at::kInt, {H, MMA, FSEQ}, dev, op, "accum_group_ids");
  expect_tensor(acc_tpg, at::kFloat, {H, MMA, MTPA}, dev, op, "accum_tokens_per_group");
  expect_tensor(acc_ng, at::kInt, {H, MMA}, dev, op, "accum_num_groups");
  if (acc_wsum) expect_tensor(*acc_wsum, at::kFloat, {H, MMA}, dev, op, "accum_weight_sum");
  expect_tensor(mk, at::kBFloat16, {H, MMB, MTPA, D}, dev, op, "merge_k_pool");
  expect_tensor(mv, at::kBFloat16, {H, MMB, MTPA, D}, dev, op, "merge_v_pool");
  expect_tensor(mpos, at::kLong, {H, MMB, MTPA, 3}, dev, op, "merge_pos_pool");
  expect_tensor(mtc, at::kInt, {H, MMB}, dev, op, "merge_token_count");
}

// ---------------------------------------------------------------------------
// PyramidKVCacheManager (pyramidkv_manager.h:62-199, .cc:36-214)
// ---------------------------------------------------------------------------
class PyramidKVCacheManager : public torch::CustomClassHolder {
 public:
  PyramidKVCacheManager(int64_t num_layers, int64_t num_heads, int64_t head_dim, int64_t frame_seqlen,
                        int64_t max_sink_frames, int64_t max_middle_frames, int64_t max_recent_frames,
                        const std::string &device_str, const std::string &kv_dtype_str, int64_t max_attend_chunks)
      : L_(num_layers), H_(num_heads), D_(head_dim), F_(frame_seqlen), ms_(max_sink_frames),
        mm_(max_middle_frames), mr_(max_recent_frames), mac_(max_attend_chunks) {
    TORCH_CHECK(num_layers > 0 && num_heads > 0 && head_dim > 0,
                "PyramidKVCacheManager: num_layers/num_heads/head_dim must be > 0");
    TORCH_CHECK(frame_seqlen > 0, "PyramidKVCacheManager: frame_seqlen must be > 0");
    TORCH_CHECK(max_sink_frames >= 0 && max_middle_frames >= 0 && max_recent_frames >= 0,
                "PyramidKVCacheManager: max_*_frames must be >= 0");
    TORCH_CHECK(max_attend_chunks > 0,
                "PyramidKVCacheManager: max_attend_chunks must be > 0 (usually = num_frame_per_block with "
                "safety margin)");
    at::ScalarType kv;
    if (kv_dtype_str == "bfloat16" || kv_dtype_str == "bf16")
      kv = at::kBFloat16;
    else if (kv_dtype_str == "float16" || kv_dtype_str == "half" || kv_dtype_str == "fp16")
      kv = at::kHalf;
    else if (kv_dtype_str == "float32" || kv_dtype_str == "float" || kv_dtype_str == "fp32")
      kv = at::kFloat;
    else
      TORCH_CHECK(false, "PyramidKVCacheManager: unsupported kv dtype '", kv_dtype_str, "'");
    const c10::Device dev(device_str);
    auto o_kv = at::TensorOptions().dtype(kv).device(dev);
    auto o64 = at::TensorOptions().dtype(at::kLong).device(dev);
    auto o32 = at::TensorOptions().dtype(at::kInt).device(dev);
    auto o8 = at::TensorOptions().dtype(at::kChar).device(dev);
    auto of = at::TensorOptions().dtype(at::kFloat).device(dev);
    const int64_t L = L_, H = H_, D = D_, F = F_;
    sink_k_ = at::zeros({L, H, ms_, F, D}, o_kv);
    sink_v_ = at::zeros({L, H, ms_, F, D}, o_kv);
    middle_k_ = at::zeros({L, H, mm_, F, D}, o_kv);
    middle_v_ = at::zeros({L, H, mm_, F, D}, o_kv);
    recent_k_ = at::zeros({L, H, mr_, F, D}, o_kv);
    recent_v_ = at::zeros({L, H, mr_, F, D}, o_kv);
    sink_pos_ = at::zeros({L, H, ms_, F, 3}, o64);
    middle_pos_ = at::zeros({L, H, mm_, F, 3}, o64);
    recent_pos_ = at::zeros({L, H, mr_, F, 3}, o64);
    head_t_ = at::full({L, H, max_total()}, -1, o64);
    write_idx_ = at::zeros({L, H, 3}, o64);
    valid_count_ = at::zeros({L, H, 3}, o64);
    strategy_ = at::zeros({L, H, 8}, o8);
    const int64_t pt = max_pack_tokens();
    k_flat_ = at::zeros({pt, 1, D}, o_kv);
    v_flat_ = at::zeros({pt, 1, D}, o_kv);
    cu_ = at::zeros({mac_ * H + 1}, o32);
    pos_flat_ = at::zeros({pt, 3}, o64);
    const int64_t MMB = kMaxMergeBlocks, MMA = kMaxMergeActive, MT = kMaxMergeTokens;
    merge_k_ = at::zeros({L, H, MMB, MT, D}, o_kv);
    merge_v_ = at::zeros({L, H, MMB, MT, D}, o_kv);
    merge_pos_ = at::zeros({L, H, MMB, MT, 3}, o64);
    merge_tc_ = at::zeros({L, H, MMB}, o32);
    acc_k_ = at::zeros({L, H, MMA, MT, D}, of);
    acc_v_ = at::zeros({L, H, MMA, MT, D}, of);
    acc_pos_ = at::zeros({L, H, MMA, MT, 3}, o64);
    acc_gid_ = at::zeros({L, H, MMA, F}, o32);
    acc_tpg_ = at::zeros({L, H, MMA, MT}, of);
    acc_ng_ = at::zeros({L, H, MMA}, o32);
    acc_wsum_ = at::zeros({L, H, MMA}, of);
  }

  void reset() {  // pyramidkv_manager.cc:160-179
    write_idx_.zero_();
    valid_count_.zero_();
    head_t_.fill_(-1);
    cu_.zero_();
    sink_pos_.zero_();
    middle_pos_.zero_();
    recent_pos_.zero_();
    merge_tc_.zero_();
    acc_ng_.zero_();
  }

  void set_strategy(int64_t layer_idx, int64_t head_idx, int64_t kind, Tensor params) {  // .cc:181-214
    TORCH_CHECK(layer_idx >= 0 && layer_idx < L_, "PyramidKVCacheManager::set_strategy layer_idx out of range");
    TORCH_CHECK(head_idx >= 0 && head_idx < H_, "PyramidKVCacheManager::set_strategy head_idx out of range");
    TORCH_CHECK(params.dtype() == at::kChar, "PyramidKVCacheManager::set_strategy params must be int8");
    TORCH_CHECK(params.dim() == 1, "params must be 1D");
    TORCH_CHECK(params.size(0) <= 7, "params longer than 7 (slot[0] is kind)");
    TORCH_CHECK(kind >= -128 && kind <= 127, "kind out of int8 range");
    auto cpu = params.to(at::kCPU).contiguous();
    auto buf = at::zeros({8}, at::TensorOptions().dtype(at::kChar));
    buf.data_ptr<int8_t>()[0] = static_cast<int8_t>(kind);
    if (cpu.size(0) > 0) std::memcpy(buf.data_ptr<int8_t>() + 1, cpu.data_ptr<int8_t>(), cpu.size(0));
    strategy_.index_put_({layer_idx, head_idx}, buf.to(strategy_.device()));
  }

  int64_t num_layers() const { return L_; }
  int64_t num_heads() const { return H_; }
  int64_t head_dim() const { return D_; }
  int64_t frame_seqlen() const { return F_; }
  int64_t max_sink() const { return ms_; }
  int64_t max_middle() const { return mm_; }
  int64_t max_recent() const { return mr_; }
  int64_t max_total() const { return ms_ + mm_ + mr_; }
  int64_t max_attend_chunks() const { return mac_; }
  int64_t max_pack_tokens() const { return mac_ * H_ * (max_total() + kMaxMergeBlocks) * F_; }
  int64_t max_total_tokens() const { return max_pack_tokens(); }
  int64_t max_merge_blocks() const { return kMaxMergeBlocks; }
  int64_t max_merge_active() const { return kMaxMergeActive; }
  int64_t max_merge_tokens_per_anchor() const { return kMaxMergeTokens; }

  Tensor sink_k_pool() const { return sink_k_; }
  Tensor sink_v_pool() const { return sink_v_; }
  Tensor middle_k_pool() const { return middle_k_; }
  Tensor middle_v_pool() const { return middle_v_; }
  Tensor recent_k_pool() const { return recent_k_; }
  Tensor recent_v_pool() const { return recent_v_; }
  Tensor sink_pos_pool() const { return sink_pos_; }
  Tensor middle_pos_pool() const { return middle_pos_; }
  Tensor recent_pos_pool() const { return recent_pos_; }
  Tensor head_t_table() const { return head_t_; }
  Tensor write_idx() const { return write_idx_; }
  Tensor valid_count() const { return valid_count_; }
  Tensor strategy() const { return strategy_; }
  Tensor k_flat_out() const { return k_flat_; }
  Tensor v_flat_out() const { return v_flat_; }
  Tensor cu_seqlens_k() const { return cu_; }
  Tensor pos_flat_out() const { return pos_flat_; }
  Tensor merge_k_pool() const { return merge_k_; }
  Tensor merge_v_pool() const { return merge_v_; }
  Tensor merge_pos_pool() const { return merge_pos_; }
  Tensor merge_token_count() const { return merge_tc_; }
  Tensor merge_accum_sum_k() const { return acc_k_; }
  Tensor merge_accum_sum_v() const { return acc_v_; }
  Tensor merge_accum_pos() const { return acc_pos_; }
  Tensor merge_accum_group_ids() const { return acc_gid_; }
  Tensor merge_accum_tokens_per_group() const { return acc_tpg_; }
  Tensor merge_accum_num_groups() const { return acc_ng_; }
  Tensor merge_accum_weight_sum() const { return acc_wsum_; }

  pkv_geometry geometry() const {
    pkv_geometry g;
    g.num_layers = static_cast<int32_t>(L_);
    g.num_heads = static_cast<int32_t>(H_);
    g.head_dim = static_cast<int32_t>(D_);
    g.frame_seqlen = static_cast<int32_t>(F_);
    g.max_sink = static_cast<int32_t>(ms_);
    g.max_middle = static_cast<int32_t>(mm_);
    g.max_recent = static_cast<int32_t>(mr_);
    g.max_merge_blocks = kMaxMergeBlocks;
    g.max_merge_active = kMaxMergeActive;
    g.max_merge_tokens = kMaxMergeTokens;
    g.max_pack_tokens = max_pack_tokens();
    return g;
  }

  pkv_pools pools() const {
    pkv_pools p;
    auto u16 = [](const Tensor &t) { return reinterpret_cast<uint16_t *>(t.data_ptr()); };
    p.sink_k = u16(sink_k_); p.sink_v = u16(sink_v_);
    p.middle_k = u16(middle_k_); p.middle_v = u16(middle_v_);
    p.recent_k = u16(recent_k_); p.recent_v = u16(recent_v_);
    p.sink_pos = sink_pos_.data_ptr<int64_t>();
    p.middle_pos = middle_pos_.data_ptr<int64_t>();
    p.recent_pos = recent_pos_.data_ptr<int64_t>();
    p.merge_k = u16(merge_k_); p.merge_v = u16(merge_v_);
    p.merge_pos = merge_pos_.data_ptr<int64_t>();
    p.merge_token_count = merge_tc_.data_ptr<int32_t>();
    p.merge_accum_sum_k = acc_k_.data_ptr<float>();
    p.merge_accum_sum_v = acc_v_.data_ptr<float>();
    p.merge_accum_pos = acc_pos_.data_ptr<int64_t>();
    p.merge_accum_group_ids = acc_gid_.data_ptr<int32_t>();
    p.merge_accum_tokens_per_group = acc_tpg_.data_ptr<float>();
    p.merge_accum_num_groups = acc_ng_.data_ptr<int32_t>();
    p.merge_accum_weight_sum = acc_wsum_.data_ptr<float>();
    p.valid_count = valid_count_.data_ptr<int64_t>();
    p.k_flat_out = u16(k_flat_); p.v_flat_out = u16(v_flat_);
    p.pos_flat_out = pos_flat_.data_ptr<int64_t>();
    return p;
  }

  void require_bf16(const char *who) const {
    TORCH_CHECK(sink_k_.scalar_type() == at::kBFloat16, who, " currently only implements bf16 pools");
  }

  // Workspace of the fused update for F frames; its first 8 [H*F] int32
  // arrays are the state-machine descriptors of the last call.
  Tensor update_workspace(int64_t frames) {
    const pkv_geometry g = geometry();
    const int64_t bytes = pkv_cache_update_workspace_size(&g, static_cast<int32_t>(frames));
    if (!ws_.defined() || ws_frames_ != frames) {
      ws_ = at::zeros({bytes}, at::TensorOptions().dtype(at::kByte).device(valid_count_.device()));
      ws_frames_ = frames;
    }
    return ws_;
  }

  // Plan buffers of the fused plan + pack, sized for max_attend_chunks;
  // cu_seqlens_k is the manager's own cu tensor.
  pkv_plan_out plan_workspace() {
    if (!pw_kind_.defined()) {
      const int64_t n = mac_ * H_ * (max_total() + kMaxMergeBlocks);
      auto o32 = at::TensorOptions().dtype(at::kInt).device(valid_count_.device());
      auto o64 = at::TensorOptions().dtype(at::kLong).device(valid_count_.device());
      pw_kind_ = at::empty({n}, o32);
      pw_sg_ = at::empty({n}, o32);
      pw_len_ = at::empty({n}, o32);
      pw_dst_ = at::empty({n}, o32);
      pw_traw_ = at::empty({n}, o64);
      pw_tremap_ = at::empty({n}, o64);
    }
    return pkv_plan_out{cu_.data_ptr<int32_t>(), pw_kind_.data_ptr<int32_t>(), pw_sg_.data_ptr<int32_t>(),
                        pw_len_.data_ptr<int32_t>(), pw_dst_.data_ptr<int32_t>(), pw_traw_.data_ptr<int64_t>(),
                        pw_tremap_.data_ptr<int64_t>()};
  }

  std::vector<Tensor> update_descriptors(int64_t frames) {
    Tensor ws = update_workspace(frames);
    const int64_t n = H_ * frames;
    const int64_t stride = (n * 4 + 255) / 256 * 256;
    std::vector<Tensor> out;
    for (int i = 0; i < 8; ++i)
      out.push_back(ws.narrow(0, i * stride, n * 4).view(at::kInt));
    return out;
  }

 private:
  int64_t L_, H_, D_, F_, ms_, mm_, mr_, mac_;
  Tensor sink_k_, sink_v_, middle_k_, middle_v_, recent_k_, recent_v_;
  Tensor sink_pos_, middle_pos_, recent_pos_, head_t_, write_idx_, valid_count_, strategy_;
  Tensor k_flat_, v_flat_, cu_, pos_flat_;
  Tensor merge_k_, merge_v_, merge_pos_, merge_tc_;
  Tensor acc_k_, acc_v_, acc_pos_, acc_gid_, acc_tpg_, acc_ng_, acc_wsum_;
  Tensor ws_;
  int64_t ws_frames_ = -1;
  Tensor pw_kind_, pw_sg_, pw_len_, pw_dst_, pw_traw_, pw_tremap_;
};

using Mgr = c10::intrusive_ptr<PyramidKVCacheManager>;

static pkv_rope_tables *rope_tables_or_null(const Tensor &ft, const Tensor &fy, const Tensor &fx,
                                            pkv_rope_tables &out, const char *who) {
  const bool any = (ft.defined() && ft.numel() > 0) || (fy.defined() && fy.numel() > 0) ||
                   (fx.defined() && fx.numel() > 0);
  if (!any) return nullptr;
  TORCH_CHECK(ft.numel() > 0 && fy.numel() > 0 && fx.numel() > 0, who,
              ": the t, y and x frequency tables must be given together");
  for (const Tensor *t : {&ft, &fy, &fx}) {
    TORCH_CHECK(t->dim() == 2 && t->scalar_type() == at::kFloat && t->is_contiguous(), who,
                ": freqs_*_flat must be contiguous 2D fp32");
  }
  out.ft = ft.data_ptr<float>();
  out.fy = fy.data_ptr<float>();
  out.fx = fx.data_ptr<float>();
  out.ft_rows = static_cast<int32_t>(ft.size(0));
  out.ft_cols = static_cast<int32_t>(ft.size(1) / 2);
  out.fy_rows = static_cast<int32_t>(fy.size(0));
  out.fy_cols = static_cast<int32_t>(fy.size(1) / 2);
  out.fx_rows = static_cast<int32_t>(fx.size(0));
  out.fx_cols = static_cast<int32_t>(fx.size(1) / 2);
  return &out;
}

// ---------------------------------------------------------------------------
// ops of the reference schema
// ---------------------------------------------------------------------------
static void pyramidkv_pack(Mgr mgr, Tensor src_kind, Tensor src_slot_global, Tensor seg_lengths,
                           Tensor dst_token_offsets, Tensor anchor_t_remap, Tensor freqs_ft_flat,
                           Tensor freqs_fy_flat, Tensor freqs_fx_flat) {
  TORCH_CHECK(mgr.get() != nullptr, "pyramidkv_pack: manager is null");
  mgr->require_bf16("pyramidkv_pack");
  TORCH_CHECK(src_kind.dtype() == at::kInt && src_slot_global.dtype() == at::kInt &&
                  seg_lengths.dtype() == at::kInt && dst_token_offsets.dtype() == at::kInt,
              "all PlanInfo descriptor tensors must be int32");
  const int64_t n = src_kind.numel();
  if (n == 0) return;
  TORCH_CHECK(src_slot_global.numel() == n && seg_lengths.numel() == n && dst_token_offsets.numel() == n,
              "pyramidkv_pack: descriptor lengths differ");
  auto sk = src_kind.contiguous(), sg = src_slot_global.contiguous(), sl = seg_lengths.contiguous(),
       dst = dst_token_offsets.contiguous();
  Tensor tr;
  if (anchor_t_remap.defined() && anchor_t_remap.numel() > 0) {
    TORCH_CHECK(anchor_t_remap.scalar_type() == at::kLong, "pyramidkv_pack: anchor_t_remap must be int64");
    TORCH_CHECK(anchor_t_remap.numel() >= n, "pyramidkv_pack: anchor_t_remap shorter than the descriptors");
    tr = anchor_t_remap.contiguous();
  }
  pkv_rope_tables rt;
  pkv_rope_tables *rope = rope_tables_or_null(freqs_ft_flat, freqs_fy_flat, freqs_fx_flat, rt, "pyramidkv_pack");
  const pkv_geometry g = mgr->geometry();
  const pkv_pools p = mgr->pools();
  pkv_check(pkv_pack(&g, &p, sk.data_ptr<int32_t>(), sg.data_ptr<int32_t>(), sl.data_ptr<int32_t>(),
                     dst.data_ptr<int32_t>(), static_cast<int32_t>(n), ptr_or_null<int64_t>(tr),
                     tr.defined() ? rope : nullptr, stream_for(sk)),
            "pyramidkv_pack");
}

static void pyramidkv_update(Mgr mgr, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor dst_kind,
                             Tensor dst_slot_global, Tensor src_frame_in_block, Tensor src_head) {
  TORCH_CHECK(mgr.get() != nullptr, "pyramidkv_update: manager is null");
  TORCH_CHECK(new_k.is_cuda() && new_v.is_cuda(), "pyramidkv_update: new_k/new_v must be on CUDA");
  TORCH_CHECK(new_k.scalar_type() == at::kBFloat16, "pyramidkv_update currently only implements bf16");
  TORCH_CHECK(dst_kind.dtype() == at::kInt && dst_slot_global.dtype() == at::kInt &&
                  src_frame_in_block.dtype() == at::kInt && src_head.dtype() == at::kInt,
              "all descriptor tensors must be int32");
  mgr->require_bf16("pyramidkv_update");
  const int64_t n = dst_kind.numel();
  if (n == 0) return;
  TORCH_CHECK(new_k.dim() == 4 && new_k.size(1) == mgr->num_heads() && new_k.size(2) == mgr->frame_seqlen() &&
                  new_k.size(3) == mgr->head_dim() && new_v.sizes() == new_k.sizes(),
              "pyramidkv_update: new_k/new_v must be [F, H, frame_seqlen, head_dim]");
  auto nk = new_k.contiguous(), nv = new_v.contiguous();
  Tensor np;
  if (new_pos.defined() && new_pos.numel() > 0) {
    TORCH_CHECK(new_pos.dtype() == at::kLong, "pyramidkv_update: new_pos must be int64");
    np = new_pos.contiguous();
  }
  auto a = dst_kind.contiguous(), b = dst_slot_global.contiguous(), c = src_frame_in_block.contiguous(),
       d = src_head.contiguous();
  const pkv_geometry g = mgr->geometry();
  const pkv_pools p = mgr->pools();
  pkv_check(pkv_update_frames(&g, &p, reinterpret_cast<const uint16_t *>(nk.data_ptr()),
                              reinterpret_cast<const uint16_t *>(nv.data_ptr()), ptr_or_null<int64_t>(np),
                              static_cast<int32_t>(nk.size(0)), a.data_ptr<int32_t>(), b.data_ptr<int32_t>(),
                              c.data_ptr<int32_t>(), d.data_ptr<int32_t>(), static_cast<int32_t>(n), stream_for(nk)),
            "pyramidkv_update");
}

static void mega_state_update(Tensor states, Tensor new_t_vals, Tensor d0, Tensor d1, Tensor d2, Tensor d3,
                              Tensor d4, Tensor d5, Tensor d6, Tensor d7, int64_t num_heads,
                              int64_t frames_in_block, int64_t pass_kind) {
  TORCH_CHECK(states.is_cuda(), "mega_state_update: states must be CUDA");
  TORCH_CHECK(states.dtype() == at::kByte, "mega_state_update: states must be uint8 (raw byte buffer)");
  TORCH_CHECK(states.is_contiguous(), "mega_state_update: states must be contiguous");
  const int64_t need = num_heads * pkv_perhead_state_size();
  TORCH_CHECK(states.numel() >= need, "mega_state_update: states buffer too small (", states.numel(), " < ", need,
              ")");
  const c10::Device dev = states.device();
  TORCH_CHECK(new_t_vals.device() == dev && new_t_vals.dtype() == at::kLong &&
                  new_t_vals.numel() >= frames_in_block,
              "new_t_vals must be int64 with frames_in_block entries on the states' device");
  for (const Tensor *t : {&d0, &d1, &d2, &d3, &d4, &d5, &d6, &d7}) {
    TORCH_CHECK(t->dtype() == at::kInt, "all descriptor tensors must be int32");
    TORCH_CHECK(t->device() == dev, "descriptor tensors must be on the states' device ", dev);
    TORCH_CHECK(t->is_contiguous() && t->numel() >= num_heads * frames_in_block,
                "descriptor tensors must be contiguous with num_heads * frames_in_block entries");
  }
  if (num_heads == 0 || frames_in_block == 0) return;
  auto tv = new_t_vals.contiguous();
  pkv_state_desc desc{d0.data_ptr<int32_t>(), d1.data_ptr<int32_t>(), d2.data_ptr<int32_t>(),
                      d3.data_ptr<int32_t>(), d4.data_ptr<int32_t>(), d5.data_ptr<int32_t>(),
                      d6.data_ptr<int32_t>(), d7.data_ptr<int32_t>()};
  pkv_check(pkv_state_update(states.data_ptr<uint8_t>(), static_cast<int32_t>(num_heads), tv.data_ptr<int64_t>(),
                             static_cast<int32_t>(frames_in_block), static_cast<int32_t>(pass_kind), &desc,
                             stream_for(states)),
            "mega_state_update");
}

static int64_t mega_state_perhead_size() { return pkv_perhead_state_size(); }

using Plan7 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

static Plan7 plan_impl(const Mgr &mgr, const Tensor &states_bytes, int64_t layer_idx,
                       const std::vector<int64_t> &t_list, int64_t sink_mode_code, int64_t sink_clamp_min,
                       int64_t sink_clamp_max, int64_t decoupled_sink_lag, int64_t hist_mode_code,
                       int64_t hist_relative_t_max, double hist_soft_factor, const char *who) {
  TORCH_CHECK(mgr.get() != nullptr, who, ": manager is null");
  TORCH_CHECK(states_bytes.dtype() == at::kByte, who, ": states_bytes must be uint8");
  TORCH_CHECK(states_bytes.numel() >= mgr->num_heads() * pkv_perhead_state_size(), who,
              ": states_bytes too small for ", mgr->num_heads(), " heads");
  TORCH_CHECK(layer_idx >= 0 && layer_idx < mgr->num_layers(), who, ": layer_idx out of range");
  const auto dev = mgr->valid_count().device();
  Tensor sb = states_bytes.to(dev).contiguous();
  const int64_t C = static_cast<int64_t>(t_list.size());
  const int64_t H = mgr->num_heads();
  const int64_t S = mgr->max_total() + mgr->max_merge_blocks();
  auto o32 = at::TensorOptions().dtype(at::kInt).device(dev);
  auto o64 = at::TensorOptions().dtype(at::kLong).device(dev);
  Tensor cu = at::empty({C * H + 1}, o32), sk = at::empty({C * H * S}, o32), sg = at::empty({C * H * S}, o32),
         sl = at::empty({C * H * S}, o32), dst = at::empty({C * H * S}, o32), traw = at::empty({C * H * S}, o64),
         tremap = at::empty({C * H * S}, o64);
  pkv_plan_out out{cu.data_ptr<int32_t>(), sk.data_ptr<int32_t>(), sg.data_ptr<int32_t>(),
                   sl.data_ptr<int32_t>(), dst.data_ptr<int32_t>(), traw.data_ptr<int64_t>(),
                   tremap.data_ptr<int64_t>()};
  pkv_remap rm{static_cast<int32_t>(sink_mode_code), static_cast<int32_t>(sink_clamp_min),
               static_cast<int32_t>(sink_clamp_max), static_cast<int32_t>(decoupled_sink_lag),
               static_cast<int32_t>(hist_mode_code), static_cast<int32_t>(hist_relative_t_max), hist_soft_factor};
  const pkv_geometry g = mgr->geometry();
  Tensor vc = mgr->valid_count().select(0, layer_idx);
  Tensor mtc = mgr->merge_token_count().select(0, layer_idx);
  int rc = pkv_plan_multi(&g, sb.data_ptr<uint8_t>(), vc.data_ptr<int64_t>(), mtc.data_ptr<int32_t>(), t_list.data(),
                          static_cast<int32_t>(C), &rm, &out, nullptr, stream_for(vc));
  if (rc == PKV_ERR_CAPACITY) TORCH_CHECK(false, "mega_plan_multi: ", pkv_last_error(), " (currently ",
                                          mgr->max_attend_chunks(), ")");
  pkv_check(rc, who);
  return {cu, sk, sg, sl, dst, traw, tremap};
}

static Plan7 mega_plan(Mgr mgr, Tensor states_bytes, int64_t layer_idx, int64_t current_t, int64_t pass_kind,
                       int64_t sink_mode_code, int64_t sink_clamp_min, int64_t sink_clamp_max,
                       int64_t decoupled_sink_lag, int64_t hist_mode_code, int64_t hist_relative_t_max,
                       double hist_soft_factor) {
  (void)pass_kind;  // reserved: the plan is the same for noisy and clean (mega_plan.cc:309)
  return plan_impl(mgr, states_bytes, layer_idx, {current_t}, sink_mode_code, sink_clamp_min, sink_clamp_max,
                   decoupled_sink_lag, hist_mode_code, hist_relative_t_max, hist_soft_factor, "mega_plan");
}

static Plan7 mega_plan_multi(Mgr mgr, Tensor states_bytes, int64_t layer_idx, Tensor current_t_list,
                             int64_t pass_kind, int64_t sink_mode_code, int64_t sink_clamp_min,
                             int64_t sink_clamp_max, int64_t decoupled_sink_lag, int64_t hist_mode_code,
                             int64_t hist_relative_t_max, double hist_soft_factor) {
  (void)pass_kind;
  TORCH_CHECK(current_t_list.dtype() == at::kLong, "mega_plan_multi: current_t_list must be int64");
  TORCH_CHECK(current_t_list.dim() == 1, "mega_plan_multi: current_t_list must be 1D");
  TORCH_CHECK(current_t_list.numel() > 0, "mega_plan_multi: empty current_t_list");
  auto tl = current_t_list.to(at::kCPU).contiguous();
  std::vector<int64_t> v(tl.data_ptr<int64_t>(), tl.data_ptr<int64_t>() + tl.numel());
  return plan_impl(mgr, states_bytes, layer_idx, v, sink_mode_code, sink_clamp_min, sink_clamp_max,
                   decoupled_sink_lag, hist_mode_code, hist_relative_t_max, hist_soft_factor, "mega_plan_multi");
}

static void merge_impl(Tensor states, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor dk, Tensor ds, Tensor df,
                       Tensor dn, Tensor acc_k, Tensor acc_v, Tensor acc_pos, Tensor acc_gid, Tensor acc_tpg,
                       Tensor acc_ng, Tensor mk, Tensor mv, Tensor mpos, Tensor mtc, const Tensor *weights,
                       const Tensor *wsum) {
  TORCH_CHECK(new_k.is_cuda() && new_v.is_cuda() && new_pos.is_cuda(), "mega_merge_accum: new_k/v/pos must be CUDA");
  TORCH_CHECK(new_k.dtype() == at::kBFloat16, "mega_merge_accum: new_k must be bf16");
  TORCH_CHECK(new_v.dtype() == at::kBFloat16, "mega_merge_accum: new_v must be bf16");
  TORCH_CHECK(new_pos.dtype() == at::kLong, "mega_merge_accum: new_pos must be int64");
  TORCH_CHECK(acc_k.dtype() == at::kFloat && acc_v.dtype() == at::kFloat, "mega_merge_accum: accumulators must be fp32");
  TORCH_CHECK(mk.dtype() == at::kBFloat16 && mv.dtype() == at::kBFloat16,
              "mega_merge_accum: merge_k/v_pool must be bf16");
  TORCH_CHECK(new_k.dim() == 4 && new_v.sizes() == new_k.sizes(), "mega_merge_accum: new_k/new_v must be [F,H,FSEQ,D]");
  const int64_t F = new_k.size(0), H = new_k.size(1), FSEQ = new_k.size(2), D = new_k.size(3);
  TORCH_CHECK(new_pos.dim() == 4 && new_pos.size(0) == F && new_pos.size(1) == H && new_pos.size(2) == FSEQ &&
                  new_pos.size(3) == 3,
              "mega_merge_accum: new_pos must be [F,H,FSEQ,3]");
  const c10::Device dev = new_k.device();
  TORCH_CHECK(new_v.device() == dev && new_pos.device() == dev, "mega_merge_accum: new_k/v/pos on different devices");
  expect_merge_layer("mega_merge_accum", dev, H, FSEQ, D, acc_k, acc_v, acc_pos, acc_gid, acc_tpg, acc_ng, wsum, mk,
                     mv, mpos, mtc);
  const int64_t MMA = acc_k.size(1), MMB = mk.size(1), MTPA = acc_k.size(2);
  TORCH_CHECK(states.device() == dev && states.dtype() == at::kByte &&
                  states.numel() >= H * pkv_perhead_state_size(),
              "mega_merge_accum: states must hold H PerHeadState records on the frames' device");
  for (const Tensor *t : {&dk, &ds, &df, &dn}) {
    TORCH_CHECK(t->device() == dev && t->scalar_type() == at::kInt && t->numel() >= H * F,
                "mega_merge_accum: descriptor tensors must be int32 on ", dev, " with at least H * F = ", H * F,
                " entries");
  }
  if (H == 0 || F == 0) return;
  auto nk = new_k.contiguous(), nv = new_v.contiguous(), np = new_pos.contiguous();
  auto k0 = dk.contiguous(), k1 = ds.contiguous(), k2 = df.contiguous(), k3 = dn.contiguous();
  for (const Tensor *t : {&k0, &k1, &k2, &k3}) check_i32(*t, "merge descriptors");
  TORCH_CHECK(!weights || weights->numel() == F, "mega_merge_accum_weighted: one weight per frame");
  Tensor st = states.contiguous();
  Tensor ws = at::empty({pkv_merge_workspace_size(H, F, FSEQ, MTPA)},
                        at::TensorOptions().dtype(at::kByte).device(nk.device()));
  pkv_merge_layer ml{acc_k.data_ptr<float>(), acc_v.data_ptr<float>(), acc_pos.data_ptr<int64_t>(),
                     acc_gid.data_ptr<int32_t>(), acc_tpg.data_ptr<float>(), acc_ng.data_ptr<int32_t>(),
                     wsum ? wsum->data_ptr<float>() : nullptr, reinterpret_cast<uint16_t *>(mk.data_ptr()),
                     reinterpret_cast<uint16_t *>(mv.data_ptr()), mpos.data_ptr<int64_t>(), mtc.data_ptr<int32_t>()};
  Tensor w;
  if (weights) w = weights->to(nk.device(), at::kFloat).contiguous();
  pkv_check(pkv_merge_accum(st.data_ptr<uint8_t>(), H, F, FSEQ, D, MMA, MMB, MTPA,
                            reinterpret_cast<const uint16_t *>(nk.data_ptr()),
                            reinterpret_cast<const uint16_t *>(nv.data_ptr()), np.data_ptr<int64_t>(),
                            k0.data_ptr<int32_t>(), k1.data_ptr<int32_t>(), k2.data_ptr<int32_t>(),
                            k3.data_ptr<int32_t>(), weights ? w.data_ptr<float>() : nullptr, &ml, ws.data_ptr(),
                            stream_for(nk)),
            "mega_merge_accum");
}

static void mega_merge_accum(Tensor states, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor dk, Tensor ds,
                             Tensor df, Tensor dn, Tensor acc_k, Tensor acc_v, Tensor acc_pos, Tensor acc_gid,
                             Tensor acc_tpg, Tensor acc_ng, Tensor mk, Tensor mv, Tensor mpos, Tensor mtc) {
  merge_impl(states, new_k, new_v, new_pos, dk, ds, df, dn, acc_k, acc_v, acc_pos, acc_gid, acc_tpg, acc_ng, mk, mv,
             mpos, mtc, nullptr, nullptr);
}

// Weighted Veil merge: sum(w_f * x) / (count * sum(w_f)); w == 1 reproduces
// mega_merge_accum bit for bit.
static void mega_merge_accum_weighted(Tensor states, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor dk,
                                      Tensor ds, Tensor df, Tensor dn, Tensor frame_weights, Tensor acc_k,
                                      Tensor acc_v, Tensor acc_pos, Tensor acc_gid, Tensor acc_tpg, Tensor acc_ng,
                                      Tensor acc_wsum, Tensor mk, Tensor mv, Tensor mpos, Tensor mtc) {
  TORCH_CHECK(frame_weights.numel() == new_k.size(0), "mega_merge_accum_weighted: one weight per frame");
  TORCH_CHECK(acc_wsum.dtype() == at::kFloat && acc_wsum.is_contiguous(),
              "mega_merge_accum_weighted: accum_weight_sum must be contiguous fp32 [H, MMA]");
  merge_impl(states, new_k, new_v, new_pos, dk, ds, df, dn, acc_k, acc_v, acc_pos, acc_gid, acc_tpg, acc_ng, mk, mv,
             mpos, mtc, &frame_weights, &acc_wsum);
}

// Veil eviction in one launch (pkv_evict_merge): mega_state_update (clean
// pass) then the (optionally weighted) merge accumulate of the frames at
// the grid positions (t, tok / W, tok % W).
static void mega_evict_merge(Tensor states, Tensor new_t_vals, Tensor new_k, Tensor new_v, int64_t spatial_width,
                             c10::optional<Tensor> frame_weights, Tensor d0, Tensor d1, Tensor d2, Tensor d3,
                             Tensor d4, Tensor d5, Tensor d6, Tensor d7, Tensor acc_k, Tensor acc_v, Tensor acc_pos,
                             Tensor acc_gid, Tensor acc_tpg, Tensor acc_ng, Tensor acc_wsum, Tensor mk, Tensor mv,
                             Tensor mpos, Tensor mtc, Tensor workspace) {
  TORCH_CHECK(new_k.is_cuda() && new_k.dtype() == at::kBFloat16 && new_v.sizes() == new_k.sizes() &&
                  new_v.dtype() == at::kBFloat16,
              "mega_evict_merge: new_k/new_v must be CUDA bf16 of equal shape");
  TORCH_CHECK(new_k.dim() == 4, "mega_evict_merge: new_k/new_v must be [F,H,FSEQ,D]");
  const int64_t F = new_k.size(0), H = new_k.size(1), FSEQ = new_k.size(2), D = new_k.size(3);
  const c10::Device dev = new_k.device();
  TORCH_CHECK(new_v.device() == dev, "mega_evict_merge: new_k/new_v on different devices");
  TORCH_CHECK(new_t_vals.device() == dev && new_t_vals.dtype() == at::kLong && new_t_vals.numel() == F,
              "mega_evict_merge: new_t_vals must be int64 [F] on the frames' device");
  TORCH_CHECK(states.device() == dev && states.dtype() == at::kByte && states.is_contiguous() &&
                  states.numel() >= H * pkv_perhead_state_size(),
              "mega_evict_merge: states must hold H PerHeadState records on the frames' device");
  for (const Tensor *t : {&d0, &d1, &d2, &d3, &d4, &d5, &d6, &d7}) expect_desc(*t, H * F, dev, "mega_evict_merge");
  expect_merge_layer("mega_evict_merge", dev, H, FSEQ, D, acc_k, acc_v, acc_pos, acc_gid, acc_tpg, acc_ng, &acc_wsum,
                     mk, mv, mpos, mtc);
  const int64_t MMA = acc_k.size(1), MMB = mk.size(1), MTPA = acc_k.size(2);
  TORCH_CHECK(workspace.device() == dev && workspace.is_contiguous() &&
                  workspace.numel() * workspace.element_size() >= pkv_evict_merge_workspace_size(static_cast<int32_t>(H)),
              "mega_evict_merge: workspace must be a contiguous CUDA tensor of at least "
              "mega_evict_merge_workspace_size(num_heads) bytes, zero-filled before first use");
  if (H == 0 || F == 0) return;
  auto nk = new_k.contiguous(), nv = new_v.contiguous();
  auto tv = new_t_vals.contiguous();
  Tensor w;
  if (frame_weights) {
    TORCH_CHECK(frame_weights->numel() == F, "mega_evict_merge: one weight per frame");
    w = frame_weights->to(nk.device(), at::kFloat).contiguous();
  }
  pkv_state_desc desc{d0.data_ptr<int32_t>(), d1.data_ptr<int32_t>(), d2.data_ptr<int32_t>(),
                      d3.data_ptr<int32_t>(), d4.data_ptr<int32_t>(), d5.data_ptr<int32_t>(),
                      d6.data_ptr<int32_t>(), d7.data_ptr<int32_t>()};
  pkv_merge_layer ml{acc_k.data_ptr<float>(), acc_v.data_ptr<float>(), acc_pos.data_ptr<int64_t>(),
                     acc_gid.data_ptr<int32_t>(), acc_tpg.data_ptr<float>(), acc_ng.data_ptr<int32_t>(),
                     acc_wsum.data_ptr<float>(), reinterpret_cast<uint16_t *>(mk.data_ptr()),
                     reinterpret_cast<uint16_t *>(mv.data_ptr()), mpos.data_ptr<int64_t>(), mtc.data_ptr<int32_t>()};
  pkv_check(pkv_evict_merge(states.data_ptr<uint8_t>(), static_cast<int32_t>(H), static_cast<int32_t>(F),
                            static_cast<int32_t>(FSEQ), static_cast<int32_t>(D), static_cast<int32_t>(MMA),
                            static_cast<int32_t>(MMB), static_cast<int32_t>(MTPA), tv.data_ptr<int64_t>(),
                            reinterpret_cast<const uint16_t *>(nk.data_ptr()),
                            reinterpret_cast<const uint16_t *>(nv.data_ptr()), static_cast<int32_t>(spatial_width),
                            frame_weights ? w.data_ptr<float>() : nullptr, &desc, &ml, workspace.data_ptr(),
                            stream_for(nk)),
            "mega_evict_merge");
}

// Bytes of the arrival-counter workspace mega_evict_merge needs.
static int64_t mega_evict_merge_workspace_size(int64_t num_heads) {
  return pkv_evict_merge_workspace_size(static_cast<int32_t>(num_heads));
}

// ---------------------------------------------------------------------------
// ops added by this build
// ---------------------------------------------------------------------------

// Ragged-cache attention (the flash_attn_varlen_func call of
// _mega_cache.py:540-559).  q [total_q, Hq, D]; with kv_per_head k/v are
// [total_k, D] (or [total_k, 1, D]) and cu_seqlens_k has num_batches*Hq+1
// entries (sequence b*Hq+h); otherwise k/v are [total_k, Hq, D] with
// cu_seqlens_k [num_batches+1].  Returns the output shaped like q.
static Tensor ragged_attention(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k,
                               int64_t max_seqlen_q, double softmax_scale, bool kv_per_head, bool causal,
                               c10::optional<Tensor> workspace) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "ragged_attention: tensors must be on the GPU");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                  v.scalar_type() == at::kBFloat16,
              "ragged_attention: q/k/v must be bf16");
  TORCH_CHECK(!causal, "ragged_attention: causal=True is not implemented (the pyramid cache attends non-causally)");
  TORCH_CHECK(q.dim() == 3, "ragged_attention: q must be [total_q, heads, head_dim]");
  check_i32(cu_seqlens_q, "cu_seqlens_q");
  check_i32(cu_seqlens_k, "cu_seqlens_k");
  const int64_t Hq = q.size(1), D = q.size(2);
  TORCH_CHECK(q.stride(2) == 1 && k.stride(-1) == 1 && v.stride(-1) == 1, "ragged_attention: head_dim must be dense");
  TORCH_CHECK(k.strides() == v.strides() && k.sizes() == v.sizes(), "ragged_attention: k and v must share a layout");
  const int64_t B = cu_seqlens_q.numel() - 1;
  TORCH_CHECK(B >= 0, "ragged_attention: cu_seqlens_q must have at least one entry");
  int64_t kv_tok = k.stride(0), kv_head = 0;
  if (kv_per_head) {
    TORCH_CHECK(cu_seqlens_k.numel() == B * Hq + 1, "ragged_attention: per-head KV needs num_batches*heads+1 "
                                                    "cu_seqlens_k entries");
    TORCH_CHECK(k.size(-1) == D && (k.dim() == 2 || (k.dim() == 3 && k.size(1) == 1)),
                "ragged_attention: per-head k/v must be [total_k, D] or [total_k, 1, D]");
  } else {
    TORCH_CHECK(cu_seqlens_k.numel() == B + 1, "ragged_attention: cu_seqlens_k must have num_batches+1 entries");
    TORCH_CHECK(k.dim() == 3 && k.size(1) == Hq && k.size(2) == D, "ragged_attention: k/v must be [total_k, H, D]");
    kv_head = k.stride(1);
  }
  Tensor out = at::empty_like(q, at::MemoryFormat::Contiguous);
  if (B == 0 || q.size(0) == 0) return out;
  pkv_attn_args a;
  a.q = reinterpret_cast<const uint16_t *>(q.data_ptr());
  a.k = reinterpret_cast<const uint16_t *>(k.data_ptr());
  a.v = reinterpret_cast<const uint16_t *>(v.data_ptr());
  a.o = reinterpret_cast<uint16_t *>(out.data_ptr());
  a.cu_seqlens_q = cu_seqlens_q.data_ptr<int32_t>();
  a.cu_seqlens_k = cu_seqlens_k.data_ptr<int32_t>();
  a.num_batches = static_cast<int32_t>(B);
  a.num_heads_q = static_cast<int32_t>(Hq);
  a.head_dim = static_cast<int32_t>(D);
  a.kv_per_head = kv_per_head ? 1 : 0;
  a.q_tok_stride = q.stride(0);
  a.q_head_stride = q.stride(1);
  a.kv_tok_stride = kv_tok;
  a.kv_head_stride = kv_head;
  a.o_tok_stride = out.stride(0);
  a.o_head_stride = out.stride(1);
  a.max_seqlen_q = static_cast<int32_t>(max_seqlen_q);
  a.softmax_scale = static_cast<float>(softmax_scale);
  a.causal = 0;
  if (workspace && workspace->defined() && workspace->numel() > 0) {
    const Tensor &w = *workspace;
    TORCH_CHECK(w.device() == q.device() && w.is_contiguous(),
                "ragged_attention: workspace must be a contiguous tensor on q's device");
    pkv_check(pkv_ragged_attn_fwd_ws(&a, w.data_ptr(), w.numel() * w.element_size(), stream_for(q)),
              "ragged_attention");
  } else {
    pkv_check(pkv_ragged_attn_fwd(&a, stream_for(q)), "ragged_attention");
  }
  return out;
}

// Bytes of the workspace ragged_attention splits small per-head-key launches
// with (on the current device).
static int64_t ragged_attention_workspace_size() { return pkv_ragged_attn_workspace_size(); }

static Tensor rope_apply(Tensor k, Tensor pos, Tensor ft, Tensor fy, Tensor fx) {
  TORCH_CHECK(k.is_cuda() && k.scalar_type() == at::kBFloat16 && k.dim() == 2,
              "rope_apply: k must be a CUDA bf16 [n, head_dim] tensor");
  TORCH_CHECK(pos.dtype() == at::kLong && pos.dim() == 2 && pos.size(1) == 3 && pos.size(0) == k.size(0),
              "rope_apply: pos must be int64 [n, 3]");
  pkv_rope_tables rt;
  pkv_rope_tables *rope = rope_tables_or_null(ft, fy, fx, rt, "rope_apply");
  TORCH_CHECK(rope != nullptr, "rope_apply: frequency tables are required");
  auto kc = k.contiguous();
  auto pc = pos.to(k.device()).contiguous();
  Tensor out = at::empty_like(kc);
  pkv_check(pkv_rope_apply(reinterpret_cast<const uint16_t *>(kc.data_ptr()), pc.data_ptr<int64_t>(), kc.size(0),
                           static_cast<int32_t>(kc.size(1)), rope, reinterpret_cast<uint16_t *>(out.data_ptr()),
                           stream_for(kc)),
            "rope_apply");
  return out;
}

// ---- DiT block row operations (the end-to-end rollout's model around the cache)
static const float *f32_or_null(const c10::optional<Tensor> &t, int64_t n, const Tensor &like, const char *who) {
  if (!t.has_value() || !t->defined()) return nullptr;
  TORCH_CHECK(t->is_cuda() && t->device() == like.device() && t->scalar_type() == at::kFloat && t->is_contiguous() &&
                  t->numel() == n,
              who, ": vector arguments must be contiguous fp32 of the row length on the input's device");
  return t->data_ptr<float>();
}

static Tensor dit_layer_norm(Tensor x, c10::optional<Tensor> mul, c10::optional<Tensor> add, bool mul_plus_one,
                             double eps) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() >= 1, "dit_layer_norm: x must be CUDA fp32");
  auto xc = x.contiguous();
  const int64_t C = xc.size(-1), rows = C ? xc.numel() / C : 0;
  Tensor out = at::empty(xc.sizes(), xc.options().dtype(at::kBFloat16));
  pkv_check(pkv_dit_layer_norm(xc.data_ptr<float>(), rows, static_cast<int32_t>(C), f32_or_null(mul, C, xc, "dit_layer_norm"),
                               f32_or_null(add, C, xc, "dit_layer_norm"), mul_plus_one ? 1 : 0, static_cast<float>(eps),
                               reinterpret_cast<uint16_t *>(out.data_ptr()), stream_for(xc)),
            "dit_layer_norm");
  return out;
}

static Tensor dit_rms_norm(Tensor x, c10::optional<Tensor> weight, double eps) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.stride(1) == 1,
              "dit_rms_norm: x must be a CUDA bf16 [rows, cols] tensor with dense rows");
  const int64_t rows = x.size(0), C = x.size(1);
  Tensor out = at::empty({rows, C}, x.options());
  pkv_check(pkv_dit_rms_norm(reinterpret_cast<const uint16_t *>(x.data_ptr()), x.stride(0), rows, static_cast<int32_t>(C),
                             f32_or_null(weight, C, x, "dit_rms_norm"), static_cast<float>(eps),
                             reinterpret_cast<uint16_t *>(out.data_ptr()), C, stream_for(x)),
            "dit_rms_norm");
  return out;
}

static void dit_residual_(Tensor x, Tensor y, c10::optional<Tensor> gate) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2 && x.is_contiguous(),
              "dit_residual_: x must be a contiguous CUDA fp32 [rows, cols] tensor");
  TORCH_CHECK(y.scalar_type() == at::kBFloat16 && y.dim() == 2 && y.sizes() == x.sizes() && y.stride(1) == 1 &&
                  y.device() == x.device(),
              "dit_residual_: y must be bf16 of x's shape with dense rows");
  pkv_check(pkv_dit_residual(x.data_ptr<float>(), x.size(0), static_cast<int32_t>(x.size(1)),
                             reinterpret_cast<const uint16_t *>(y.data_ptr()), y.stride(0),
                             f32_or_null(gate, x.size(1), x, "dit_residual_"), stream_for(x)),
            "dit_residual_");
}

static Tensor dit_residual_layer_norm_(Tensor x, Tensor y, c10::optional<Tensor> gate, c10::optional<Tensor> mul,
                                       c10::optional<Tensor> add, bool mul_plus_one, double eps) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2 && x.is_contiguous(),
              "dit_residual_layer_norm_: x must be a contiguous CUDA fp32 [rows, cols] tensor");
  TORCH_CHECK(y.scalar_type() == at::kBFloat16 && y.dim() == 2 && y.sizes() == x.sizes() && y.stride(1) == 1 &&
                  y.device() == x.device(),
              "dit_residual_layer_norm_: y must be bf16 of x's shape with dense rows");
  const int64_t C = x.size(1);
  Tensor out = at::empty(x.sizes(), x.options().dtype(at::kBFloat16));
  pkv_check(pkv_dit_residual_layer_norm(x.data_ptr<float>(), x.size(0), static_cast<int32_t>(C),
                                        reinterpret_cast<const uint16_t *>(y.data_ptr()), y.stride(0),
                                        f32_or_null(gate, C, x, "dit_residual_layer_norm_"),
                                        f32_or_null(mul, C, x, "dit_residual_layer_norm_"),
                                        f32_or_null(add, C, x, "dit_residual_layer_norm_"), mul_plus_one ? 1 : 0,
                                        static_cast<float>(eps), reinterpret_cast<uint16_t *>(out.data_ptr()),
                                        stream_for(x)),
            "dit_residual_layer_norm_");
  return out;
}

static Tensor dit_gelu_tanh(Tensor x) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16, "dit_gelu_tanh: x must be CUDA bf16");
  auto xc = x.contiguous();
  Tensor out = at::empty_like(xc);
  pkv_check(pkv_dit_gelu_tanh(reinterpret_cast<const uint16_t *>(xc.data_ptr()), xc.numel(),
                              reinterpret_cast<uint16_t *>(out.data_ptr()), stream_for(xc)),
            "dit_gelu_tanh");
  return out;
}

// Fused MegaCache.update for one layer (see pkv_cache_update).
static void cache_update(Mgr mgr, Tensor states_layer, Tensor sink_caps_layer, Tensor committed_vc_layer,
                         Tensor new_k, Tensor new_v, int64_t layer, int64_t t0, int64_t pass_kind,
                         int64_t shift_pending, int64_t spatial_width, int64_t merge_heads) {
  TORCH_CHECK(mgr.get() != nullptr, "cache_update: manager is null");
  mgr->require_bf16("cache_update");
  TORCH_CHECK(new_k.is_cuda() && new_k.scalar_type() == at::kBFloat16 && new_v.sizes() == new_k.sizes(),
              "cache_update: new_k/new_v must be CUDA bf16 of equal shape");
  TORCH_CHECK(new_k.dim() == 4 && new_k.size(0) == 1 && new_k.size(2) == mgr->num_heads() &&
                  new_k.size(3) == mgr->head_dim(),
              "cache_update: new_k must be [1, L_in, H, D]");
  const int64_t L_in = new_k.size(1);
  TORCH_CHECK(L_in % mgr->frame_seqlen() == 0, "cache_update: L_in (", L_in, ") not a multiple of frame_seqlen (",
              mgr->frame_seqlen(), ")");
  TORCH_CHECK(new_k.stride(3) == 1 && new_k.stride(2) == mgr->head_dim() && new_v.strides() == new_k.strides(),
              "cache_update: new_k/new_v must have dense [H, D] rows");
  const c10::Device dev = mgr->valid_count().device();
  TORCH_CHECK(new_k.device() == dev && new_v.device() == dev && states_layer.device() == dev &&
                  sink_caps_layer.device() == dev && committed_vc_layer.device() == dev,
              "cache_update: new_k/new_v, states_layer, sink_caps_layer and committed_vc_layer must be on the "
              "manager's device ", dev);
  TORCH_CHECK(states_layer.dtype() == at::kByte && states_layer.is_contiguous() &&
                  states_layer.numel() >= mgr->num_heads() * pkv_perhead_state_size(),
              "cache_update: states_layer must be contiguous uint8 [H * 600]");
  TORCH_CHECK(sink_caps_layer.dtype() == at::kLong && sink_caps_layer.is_contiguous() &&
                  sink_caps_layer.numel() == mgr->num_heads(),
              "cache_update: sink_caps_layer must be contiguous int64 [H]");
  TORCH_CHECK(committed_vc_layer.dtype() == at::kLong && committed_vc_layer.is_contiguous() &&
                  committed_vc_layer.numel() == mgr->num_heads() * 3,
              "cache_update: committed_vc_layer must be contiguous int64 [H, 3]");
  const int64_t F = L_in / mgr->frame_seqlen();
  Tensor ws = mgr->update_workspace(F);
  const pkv_geometry g = mgr->geometry();
  const pkv_pools p = mgr->pools();
  pkv_update_args a;
  a.layer = static_cast<int32_t>(layer);
  a.frames = static_cast<int32_t>(F);
  a.t0 = t0;
  a.pass_kind = static_cast<int32_t>(pass_kind);
  a.shift_pending = static_cast<int32_t>(shift_pending);
  a.spatial_width = static_cast<int32_t>(spatial_width);
  a.reserved = 0;
  a.merge_heads = static_cast<uint64_t>(merge_heads);
  a.new_k = reinterpret_cast<const uint16_t *>(new_k.data_ptr());
  a.new_v = reinterpret_cast<const uint16_t *>(new_v.data_ptr());
  a.tok_stride = new_k.stride(1);
  a.head_stride = new_k.stride(2);
  a.states_layer = states_layer.data_ptr<uint8_t>();
  a.sink_caps_layer = sink_caps_layer.data_ptr<int64_t>();
  a.committed_vc_layer = committed_vc_layer.data_ptr<int64_t>();
  a.workspace = ws.data_ptr();
  pkv_check(pkv_cache_update(&g, &p, &a, stream_for(new_k)), "cache_update");
}

static std::vector<Tensor> update_descriptors(Mgr mgr, int64_t frames) { return mgr->update_descriptors(frames); }

// ---------------------------------------------------------------------------
// data-movement ops of the _ops.py surface (scatter_copy_bind.cpp:451-683)
// and the legacy planner (pyramidkv_plan.cc:46-133)
// ---------------------------------------------------------------------------
static void check_dev_i64(const Tensor &t, const char *name, int64_t n) {
  TORCH_CHECK(t.is_cuda(), name, " must be on CUDA");
  TORCH_CHECK(t.dtype() == at::kLong, name, " must be int64");
  TORCH_CHECK(t.dim() == 1, name, " must be 1D");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.size(0) >= n, name, " is too small");
}

static void scatter_copy(Tensor src_ptrs, Tensor lengths, Tensor offsets, Tensor dst, int64_t col_dim) {
  TORCH_CHECK(src_ptrs.is_cuda(), "src_ptrs must be on CUDA");
  TORCH_CHECK(dst.is_cuda(), "dst must be on CUDA");
  TORCH_CHECK(src_ptrs.dtype() == at::kLong, "src_ptrs must be int64");
  const int64_t n = src_ptrs.size(0);
  if (n == 0) return;
  check_dev_i64(src_ptrs, "src_ptrs", n);
  check_dev_i64(lengths, "lengths", n);
  check_dev_i64(offsets, "offsets", n);
  TORCH_CHECK(dst.is_contiguous(), "dst must be contiguous");
  TORCH_CHECK(col_dim > 0, "col_dim must be > 0");
  const int64_t row_bytes = col_dim * static_cast<int64_t>(dst.element_size());
  const int64_t dst_rows = dst.numel() / col_dim;
  pkv_check(pkv_scatter_copy(src_ptrs.data_ptr<int64_t>(), lengths.data_ptr<int64_t>(), offsets.data_ptr<int64_t>(),
                             static_cast<int32_t>(n), dst.data_ptr(), dst_rows, row_bytes, stream_for(dst)),
            "scatter_copy");
}

static void apply_pos_override(Tensor pos, Tensor starts, Tensor ends, Tensor vals) {
  TORCH_CHECK(pos.is_cuda(), "pos must be on CUDA");
  TORCH_CHECK(pos.size(1) == 3, "pos must have 3 columns");
  const int64_t m = starts.size(0);
  if (m == 0) return;
  TORCH_CHECK(pos.dtype() == at::kLong && pos.is_contiguous(), "pos must be contiguous int64 [N, 3]");
  check_dev_i64(starts, "starts", m);
  check_dev_i64(ends, "ends", m);
  check_dev_i64(vals, "vals", m);
  pkv_check(pkv_pos_override(pos.data_ptr<int64_t>(), pos.size(0), starts.data_ptr<int64_t>(),
                             ends.data_ptr<int64_t>(), vals.data_ptr<int64_t>(), static_cast<int32_t>(m),
                             stream_for(pos)),
            "apply_pos_override");
}

static int32_t mapping_mode_code(const std::string &mode) {
  if (mode == "relative_clamp") return 1;
  if (mode == "relative_softcap") return 2;
  return 0;  // "none" and unknown modes (scatter_copy_bind.cpp:481-486)
}

// device pointers of the tensors -> int64 device tensor (synchronous copy
// from a host tensor, so the host buffer outlives the transfer)
static void fill_ptrs(const std::vector<Tensor> &ts, Tensor dst, const char *name) {
  std::vector<int64_t> host;
  host.reserve(ts.size());
  c10::optional<c10::Device> dev;
  for (size_t i = 0; i < ts.size(); ++i) {
    TORCH_CHECK(ts[i].is_cuda(), name, "[", i, "] must be on CUDA");
    TORCH_CHECK(ts[i].is_contiguous(), name, "[", i, "] must be contiguous");
    if (!dev) dev = ts[i].device();
    TORCH_CHECK(ts[i].device() == *dev, name, "[", i, "] is on a different CUDA device");
    host.push_back(reinterpret_cast<int64_t>(ts[i].data_ptr()));
  }
  if (host.empty()) return;
  auto cpu = at::from_blob(host.data(), {static_cast<int64_t>(host.size())}, at::TensorOptions().dtype(at::kLong));
  dst.narrow(0, 0, static_cast<int64_t>(host.size())).copy_(cpu, /*non_blocking=*/false);
}

static void refresh_readout_layout(std::vector<Tensor> src_k, std::vector<Tensor> src_v, std::vector<Tensor> src_pos,
                                   Tensor src_ptrs_k, Tensor src_ptrs_v, Tensor src_ptrs_pos, Tensor offsets,
                                   Tensor lengths, Tensor flags, Tensor dynamic_rope_t, Tensor dst_k_raw,
                                   Tensor dst_v, Tensor dst_rope_pos, Tensor dst_frame_ids, int64_t head_dim,
                                   int64_t current_t, std::string history_time_mapping_mode,
                                   int64_t history_relative_t_max, double history_time_soft_factor) {
  const int64_t n = static_cast<int64_t>(src_k.size());
  TORCH_CHECK(src_v.size() == src_k.size(), "src_v length must match src_k");
  TORCH_CHECK(src_pos.size() == src_k.size(), "src_pos length must match src_k");
  if (n == 0) return;
  TORCH_CHECK(dst_k_raw.is_cuda() && dst_v.is_cuda() && dst_rope_pos.is_cuda() && dst_frame_ids.is_cuda(),
              "refresh_readout_layout: outputs must be on CUDA");
  TORCH_CHECK(dst_rope_pos.dtype() == at::kLong, "dst_rope_pos must be int64");
  TORCH_CHECK(dst_frame_ids.dtype() == at::kLong, "dst_frame_ids must be int64");
  TORCH_CHECK(dst_k_raw.is_contiguous() && dst_v.is_contiguous() && dst_rope_pos.is_contiguous() &&
                  dst_frame_ids.is_contiguous(),
              "refresh_readout_layout: outputs must be contiguous");
  TORCH_CHECK(dst_k_raw.dtype() == dst_v.dtype(), "dst_k_raw/dst_v dtype mismatch");
  TORCH_CHECK(dst_k_raw.size(1) == head_dim, "dst_k_raw head_dim mismatch");
  TORCH_CHECK(dst_v.size(1) == head_dim, "dst_v head_dim mismatch");
  TORCH_CHECK(dst_rope_pos.size(1) == 3, "dst_rope_pos must have 3 columns");
  TORCH_CHECK(dst_v.size(0) == dst_k_raw.size(0) && dst_rope_pos.size(0) == dst_k_raw.size(0) &&
                  dst_frame_ids.size(0) >= dst_k_raw.size(0),
              "refresh_readout_layout: output row counts differ");
  for (const Tensor *t : {&src_ptrs_k, &src_ptrs_v, &src_ptrs_pos, &offsets, &lengths, &flags, &dynamic_rope_t}) {
    check_dev_i64(*t, "refresh_readout_layout descriptor", n);
    TORCH_CHECK(t->device() == dst_k_raw.device(), "descriptor device mismatch");
  }
  for (int64_t i = 0; i < n; ++i) {
    TORCH_CHECK(src_k[i].dtype() == dst_k_raw.dtype(), "src_k dtype mismatch");
    TORCH_CHECK(src_v[i].dtype() == dst_v.dtype(), "src_v dtype mismatch");
    TORCH_CHECK(src_pos[i].dtype() == at::kLong, "src_pos must be int64");
    TORCH_CHECK(src_k[i].size(1) == head_dim, "src_k head_dim mismatch");
    TORCH_CHECK(src_v[i].size(1) == head_dim, "src_v head_dim mismatch");
    TORCH_CHECK(src_pos[i].size(1) == 3, "src_pos must have 3 columns");
    TORCH_CHECK(src_k[i].device() == dst_k_raw.device(), "src_k device mismatch");
  }
  fill_ptrs(src_k, src_ptrs_k, "src_k");
  fill_ptrs(src_v, src_ptrs_v, "src_v");
  fill_ptrs(src_pos, src_ptrs_pos, "src_pos");
  pkv_refresh_args a;
  a.src_ptrs_k = src_ptrs_k.data_ptr<int64_t>();
  a.src_ptrs_v = src_ptrs_v.data_ptr<int64_t>();
  a.src_ptrs_pos = src_ptrs_pos.data_ptr<int64_t>();
  a.offsets = offsets.data_ptr<int64_t>();
  a.lengths = lengths.data_ptr<int64_t>();
  a.flags = flags.data_ptr<int64_t>();
  a.dynamic_rope_t = dynamic_rope_t.data_ptr<int64_t>();
  a.dst_k = dst_k_raw.data_ptr();
  a.dst_v = dst_v.data_ptr();
  a.dst_pos = dst_rope_pos.data_ptr<int64_t>();
  a.dst_frame_ids = dst_frame_ids.data_ptr<int64_t>();
  a.dst_rows = dst_k_raw.size(0);
  a.row_bytes = head_dim * static_cast<int64_t>(dst_k_raw.element_size());
  a.current_t = current_t;
  a.history_relative_t_max = history_relative_t_max;
  a.n_segments = static_cast<int32_t>(n);
  a.history_mode_code = mapping_mode_code(history_time_mapping_mode);
  a.history_soft_factor = static_cast<float>(history_time_soft_factor);
  pkv_check(pkv_refresh_readout(&a, stream_for(dst_k_raw)), "refresh_readout_layout");
}

static void anchor_store_write_frames(Tensor k_seq, Tensor v_seq, Tensor pos_seq, Tensor frame_desc, Tensor store_k,
                                      Tensor store_v, Tensor store_pos) {
  for (const Tensor *t : {&k_seq, &v_seq, &pos_seq, &frame_desc, &store_k, &store_v, &store_pos}) {
    TORCH_CHECK(t->is_cuda(), "anchor_store_write_frames: tensors must be on CUDA");
    TORCH_CHECK(t->is_contiguous(), "anchor_store_write_frames: tensors must be contiguous");
  }
  TORCH_CHECK(k_seq.dtype() == store_k.dtype(), "k_seq/store_k dtype mismatch");
  TORCH_CHECK(v_seq.dtype() == store_v.dtype(), "v_seq/store_v dtype mismatch");
  TORCH_CHECK(pos_seq.dtype() == at::kLong, "pos_seq must be int64");
  TORCH_CHECK(store_pos.dtype() == at::kLong, "store_pos must be int64");
  TORCH_CHECK(frame_desc.dtype() == at::kLong, "frame_desc must be int64");
  TORCH_CHECK(k_seq.dim() == 2, "k_seq must be [tokens, head_dim]");
  TORCH_CHECK(v_seq.dim() == 2 && v_seq.sizes() == k_seq.sizes(), "v_seq must be [tokens, head_dim]");
  TORCH_CHECK(pos_seq.dim() == 2 && pos_seq.size(1) == 3 && pos_seq.size(0) == k_seq.size(0),
              "pos_seq must be [tokens, 3]");
  TORCH_CHECK(frame_desc.dim() == 2 && frame_desc.size(1) == 2, "frame_desc must be [N, 2]");
  TORCH_CHECK(store_k.dim() == 3, "store_k must be [capacity, frame_seqlen, head_dim]");
  TORCH_CHECK(store_v.dim() == 3 && store_v.sizes() == store_k.sizes(),
              "store_v must be [capacity, frame_seqlen, head_dim]");
  TORCH_CHECK(store_pos.dim() == 3 && store_pos.size(2) == 3 && store_pos.size(0) == store_k.size(0) &&
                  store_pos.size(1) == store_k.size(1),
              "store_pos must be [capacity, frame_seqlen, 3]");
  TORCH_CHECK(k_seq.size(1) == store_k.size(2), "head_dim mismatch");
  const int64_t n = frame_desc.size(0);
  if (n == 0) return;
  const int64_t fs = store_k.size(1);
  const int64_t row_bytes = store_k.size(2) * static_cast<int64_t>(store_k.element_size());
  pkv_check(pkv_anchor_store_write_frames(k_seq.data_ptr(), v_seq.data_ptr(), pos_seq.data_ptr<int64_t>(),
                                          k_seq.size(0) / fs, frame_desc.data_ptr<int64_t>(), static_cast<int32_t>(n),
                                          store_k.data_ptr(), store_v.data_ptr(), store_pos.data_ptr<int64_t>(),
                                          store_k.size(0), fs, row_bytes, stream_for(store_k)),
            "anchor_store_write_frames");
}

using Plan5 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor>;

// Legacy plan over all layers and heads (pyramidkv_plan.cc:46-133): fresh
// device tensors, built on the device from valid_count (no host round trip).
static Plan5 pyramidkv_plan(Mgr mgr, int64_t current_t, int64_t pass_kind) {
  TORCH_CHECK(mgr.get() != nullptr, "pyramidkv_plan: manager is null");
  (void)current_t;
  (void)pass_kind;
  const int64_t N = mgr->num_layers() * mgr->num_heads();
  auto o32 = at::TensorOptions().dtype(at::kInt).device(mgr->valid_count().device());
  Tensor cu = at::empty({N + 1}, o32), sk = at::empty({3 * N}, o32), sg = at::empty({3 * N}, o32),
         sl = at::empty({3 * N}, o32), dst = at::empty({3 * N}, o32);
  const pkv_geometry g = mgr->geometry();
  pkv_check(pkv_plan_legacy(&g, mgr->valid_count().data_ptr<int64_t>(), cu.data_ptr<int32_t>(),
                            sk.data_ptr<int32_t>(), sg.data_ptr<int32_t>(), sl.data_ptr<int32_t>(),
                            dst.data_ptr<int32_t>(), stream_for(cu)),
            "pyramidkv_plan");
  return {cu, sk, sg, sl, dst};
}

// MegaCache.attend's K/V side (pkv_plan_pack): plan for the chunks of
// current_t_list with layer offsets folded in, then pack (+RoPE when the
// three tables are non-empty) into the manager's flat outputs.  Returns the
// manager's cu_seqlens_k narrowed to C*H+1 entries.
static Tensor mega_attend_kv(Mgr mgr, Tensor states_layer, int64_t layer_idx, Tensor current_t_list,
                             int64_t sink_mode_code, int64_t sink_clamp_min, int64_t sink_clamp_max,
                             int64_t decoupled_sink_lag, Tensor freqs_ft_flat, Tensor freqs_fy_flat,
                             Tensor freqs_fx_flat) {
  TORCH_CHECK(mgr.get() != nullptr, "mega_attend_kv: manager is null");
  mgr->require_bf16("mega_attend_kv");
  TORCH_CHECK(states_layer.dtype() == at::kByte && states_layer.is_contiguous() &&
                  states_layer.device() == mgr->valid_count().device() &&
                  states_layer.numel() >= mgr->num_heads() * pkv_perhead_state_size(),
              "mega_attend_kv: states_layer must be a contiguous uint8 [H * 600] tensor on the manager's device");
  TORCH_CHECK(layer_idx >= 0 && layer_idx < mgr->num_layers(), "mega_attend_kv: layer_idx out of range");
  TORCH_CHECK(current_t_list.dtype() == at::kLong && current_t_list.dim() == 1 && current_t_list.numel() > 0,
              "mega_attend_kv: current_t_list must be a non-empty 1D int64 tensor");
  auto tl = current_t_list.to(at::kCPU).contiguous();
  const int64_t C = tl.numel();
  TORCH_CHECK(C <= mgr->max_attend_chunks(), "mega_attend_kv: ", C, " chunks exceed max_attend_chunks (",
              mgr->max_attend_chunks(), ")");
  pkv_rope_tables rt;
  pkv_rope_tables *rope = rope_tables_or_null(freqs_ft_flat, freqs_fy_flat, freqs_fx_flat, rt, "mega_attend_kv");
  pkv_remap rm{static_cast<int32_t>(sink_mode_code), static_cast<int32_t>(sink_clamp_min),
               static_cast<int32_t>(sink_clamp_max), static_cast<int32_t>(decoupled_sink_lag), 0, 0, 1.0};
  const pkv_geometry g = mgr->geometry();
  const pkv_pools p = mgr->pools();
  const pkv_plan_out ws = mgr->plan_workspace();
  pkv_check(pkv_plan_pack(&g, &p, states_layer.data_ptr<uint8_t>(), static_cast<int32_t>(layer_idx),
                          tl.data_ptr<int64_t>(), static_cast<int32_t>(C), &rm, rope, &ws,
                          stream_for(states_layer)),
            "mega_attend_kv");
  return mgr->cu_seqlens_k().narrow(0, 0, C * mgr->num_heads() + 1);
}

}  // namespace adahead

// ---------------------------------------------------------------------------
// meta kernels: the ops return nothing or fresh plan tensors
// ---------------------------------------------------------------------------
namespace adahead_meta {
using at::Tensor;
using adahead::Mgr;
static void pack(Mgr, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor) {}
static void update(Mgr, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor) {}
static void state_update(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, int64_t,
                         int64_t, int64_t) {}
static void merge(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                  Tensor, Tensor, Tensor, Tensor, Tensor, Tensor) {}
static void merge_w(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                    Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor) {}
static adahead::Plan7 plan_shapes(const Mgr &mgr, int64_t C) {
  const int64_t H = mgr->num_heads(), S = mgr->max_total() + mgr->max_merge_blocks();
  auto i32 = at::TensorOptions().dtype(at::kInt).device(at::kMeta);
  auto i64 = at::TensorOptions().dtype(at::kLong).device(at::kMeta);
  return {at::empty({C * H + 1}, i32), at::empty({C * H * S}, i32), at::empty({C * H * S}, i32),
          at::empty({C * H * S}, i32), at::empty({C * H * S}, i32), at::empty({C * H * S}, i64),
          at::empty({C * H * S}, i64)};
}
static adahead::Plan7 plan(Mgr mgr, Tensor, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                           int64_t, double) {
  return plan_shapes(mgr, 1);
}
static adahead::Plan7 plan_multi(Mgr mgr, Tensor, int64_t, Tensor t_list, int64_t, int64_t, int64_t, int64_t,
                                 int64_t, int64_t, int64_t, double) {
  return plan_shapes(mgr, t_list.numel());
}
static Tensor attn(Tensor q, Tensor, Tensor, Tensor, Tensor, int64_t, double, bool, bool, c10::optional<Tensor>) {
  return at::empty_like(q);
}
static Tensor rope(Tensor k, Tensor, Tensor, Tensor, Tensor) { return at::empty_like(k); }
static Tensor dit_ln(Tensor x, c10::optional<Tensor>, c10::optional<Tensor>, bool, double) {
  return at::empty(x.sizes(), x.options().dtype(at::kBFloat16));
}
static Tensor dit_rms(Tensor x, c10::optional<Tensor>, double) { return at::empty({x.size(0), x.size(1)}, x.options()); }
static void dit_residual(Tensor, Tensor, c10::optional<Tensor>) {}
static Tensor dit_gelu(Tensor x) { return at::empty_like(x); }
static Tensor dit_res_ln(Tensor x, Tensor, c10::optional<Tensor>, c10::optional<Tensor>, c10::optional<Tensor>, bool,
                         double) {
  return at::empty(x.sizes(), x.options().dtype(at::kBFloat16));
}
static void cache_update(Mgr, Tensor, Tensor, Tensor, Tensor, Tensor, int64_t, int64_t, int64_t, int64_t, int64_t,
                         int64_t) {}
static void scatter_copy(Tensor, Tensor, Tensor, Tensor, int64_t) {}
static void pos_override(Tensor, Tensor, Tensor, Tensor) {}
static void write_frames(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor) {}
static void refresh(std::vector<Tensor>, std::vector<Tensor>, std::vector<Tensor>, Tensor, Tensor, Tensor, Tensor,
                    Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, int64_t, int64_t, std::string, int64_t,
                    double) {}
}  // namespace adahead_meta

TORCH_LIBRARY(adahead, m) {
  using M = adahead::PyramidKVCacheManager;
  m.class_<M>("PyramidKVCacheManager")
      .def(torch::init<int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, const std::string &,
                       const std::string &, int64_t>())
      .def("reset", &M::reset)
      .def("set_strategy", &M::set_strategy)
      .def("sink_pool", &M::sink_k_pool)
      .def("middle_pool", &M::middle_k_pool)
      .def("recent_pool", &M::recent_k_pool)
      .def("sink_k_pool", &M::sink_k_pool)
      .def("sink_v_pool", &M::sink_v_pool)
      .def("middle_k_pool", &M::middle_k_pool)
      .def("middle_v_pool", &M::middle_v_pool)
      .def("recent_k_pool", &M::recent_k_pool)
      .def("recent_v_pool", &M::recent_v_pool)
      .def("sink_pos_pool", &M::sink_pos_pool)
      .def("middle_pos_pool", &M::middle_pos_pool)
      .def("recent_pos_pool", &M::recent_pos_pool)
      .def("head_t_table", &M::head_t_table)
      .def("write_idx", &M::write_idx)
      .def("valid_count", &M::valid_count)
      .def("strategy", &M::strategy)
      .def("k_flat_out", &M::k_flat_out)
      .def("v_flat_out", &M::v_flat_out)
      .def("cu_seqlens_k", &M::cu_seqlens_k)
      .def("pos_flat_out", &M::pos_flat_out)
      .def("merge_k_pool", &M::merge_k_pool)
      .def("merge_v_pool", &M::merge_v_pool)
      .def("merge_pos_pool", &M::merge_pos_pool)
      .def("merge_token_count", &M::merge_token_count)
      .def("merge_accum_sum_k", &M::merge_accum_sum_k)
      .def("merge_accum_sum_v", &M::merge_accum_sum_v)
      .def("merge_accum_pos", &M::merge_accum_pos)
      .def("merge_accum_group_ids", &M::merge_accum_group_ids)
      .def("merge_accum_tokens_per_group", &M::merge_accum_tokens_per_group)
      .def("merge_accum_num_groups", &M::merge_accum_num_groups)
      .def("merge_accum_weight_sum", &M::merge_accum_weight_sum)
      .def("max_merge_blocks", &M::max_merge_blocks)
      .def("max_merge_active", &M::max_merge_active)
      .def("max_merge_tokens_per_anchor", &M::max_merge_tokens_per_anchor)
      .def("num_layers", &M::num_layers)
      .def("num_heads", &M::num_heads)
      .def("head_dim", &M::head_dim)
      .def("frame_seqlen", &M::frame_seqlen)
      .def("max_sink", &M::max_sink)
      .def("max_middle", &M::max_middle)
      .def("max_recent", &M::max_recent)
      .def("max_total", &M::max_total)
      .def("max_total_tokens", &M::max_total_tokens)
      .def("max_attend_chunks", &M::max_attend_chunks)
      .def("max_pack_tokens", &M::max_pack_tokens);

  m.def("pyramidkv_pack(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor src_kind, "
        "Tensor src_slot_global, Tensor seg_lengths, Tensor dst_token_offsets, Tensor anchor_t_remap, "
        "Tensor freqs_ft_flat, Tensor freqs_fy_flat, Tensor freqs_fx_flat) -> ()");
  m.def("pyramidkv_update(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor new_k, Tensor new_v, "
        "Tensor new_pos, Tensor dst_kind, Tensor dst_slot_global, Tensor src_frame_in_block, Tensor src_head) -> ()");
  m.def("mega_state_update(Tensor(a!) states, Tensor new_t_vals, Tensor(b!) desc_dst_kind, "
        "Tensor(c!) desc_dst_slot, Tensor(d!) desc_src_frame, Tensor(e!) desc_src_head, "
        "Tensor(f!) desc_merge_accum_slot, Tensor(g!) desc_merge_local_idx, "
        "Tensor(h!) desc_merge_finalize_completed_idx, Tensor(i!) desc_merge_is_new_block, "
        "int num_heads, int frames_in_block, int pass_kind) -> ()");
  m.def("mega_plan(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor states_bytes, int layer_idx, "
        "int current_t, int pass_kind, int sink_mode_code, int sink_clamp_min, int sink_clamp_max, "
        "int decoupled_sink_lag, int hist_mode_code, int hist_relative_t_max, float hist_soft_factor) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("mega_plan_multi(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor states_bytes, "
        "int layer_idx, Tensor current_t_list, int pass_kind, int sink_mode_code, int sink_clamp_min, "
        "int sink_clamp_max, int decoupled_sink_lag, int hist_mode_code, int hist_relative_t_max, "
        "float hist_soft_factor) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("mega_state_perhead_size() -> int");
  m.def("mega_merge_accum(Tensor states, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor desc_dst_kind, "
        "Tensor desc_merge_accum_slot, Tensor desc_merge_finalize_completed_idx, Tensor desc_merge_is_new_block, "
        "Tensor(a!) accum_sum_k, Tensor(b!) accum_sum_v, Tensor(c!) accum_pos, Tensor(d!) accum_group_ids, "
        "Tensor(e!) accum_tokens_per_group, Tensor(f!) accum_num_groups, Tensor(g!) merge_k_pool, "
        "Tensor(h!) merge_v_pool, Tensor(i!) merge_pos_pool, Tensor(j!) merge_token_count) -> ()");
  m.def("mega_evict_merge(Tensor(a!) states, Tensor new_t_vals, Tensor new_k, Tensor new_v, int spatial_width, "
        "Tensor? frame_weights, Tensor(b!) desc_dst_kind, Tensor(c!) desc_dst_slot, Tensor(d!) desc_src_frame, "
        "Tensor(e!) desc_src_head, Tensor(f!) desc_merge_accum_slot, Tensor(g!) desc_merge_local_idx, "
        "Tensor(h!) desc_merge_finalize_completed_idx, Tensor(i!) desc_merge_is_new_block, Tensor(j!) accum_sum_k, "
        "Tensor(k!) accum_sum_v, Tensor(l!) accum_pos, Tensor(m!) accum_group_ids, "
        "Tensor(n!) accum_tokens_per_group, Tensor(o!) accum_num_groups, Tensor(p!) accum_weight_sum, "
        "Tensor(q!) merge_k_pool, Tensor(r!) merge_v_pool, Tensor(s!) merge_pos_pool, "
        "Tensor(t!) merge_token_count, Tensor(u!) workspace) -> ()");
  m.def("mega_evict_merge_workspace_size(int num_heads) -> int");
  m.def("mega_merge_accum_weighted(Tensor states, Tensor new_k, Tensor new_v, Tensor new_pos, Tensor desc_dst_kind, "
        "Tensor desc_merge_accum_slot, Tensor desc_merge_finalize_completed_idx, Tensor desc_merge_is_new_block, "
        "Tensor frame_weights, Tensor(a!) accum_sum_k, Tensor(b!) accum_sum_v, Tensor(c!) accum_pos, "
        "Tensor(d!) accum_group_ids, Tensor(e!) accum_tokens_per_group, Tensor(f!) accum_num_groups, "
        "Tensor(g!) accum_weight_sum, Tensor(h!) merge_k_pool, Tensor(i!) merge_v_pool, "
        "Tensor(j!) merge_pos_pool, Tensor(k!) merge_token_count) -> ()");
  m.def("ragged_attention(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
        "int max_seqlen_q, float softmax_scale, bool kv_per_head=True, bool causal=False, "
        "Tensor? workspace=None) -> Tensor");
  m.def("ragged_attention_workspace_size() -> int");
  m.def("rope_apply(Tensor k, Tensor pos, Tensor freqs_ft_flat, Tensor freqs_fy_flat, Tensor freqs_fx_flat) "
        "-> Tensor");
  m.def("dit_layer_norm(Tensor x, Tensor? mul, Tensor? add, bool mul_plus_one, float eps) -> Tensor");
  m.def("dit_rms_norm(Tensor x, Tensor? weight, float eps) -> Tensor");
  m.def("dit_residual_(Tensor(a!) x, Tensor y, Tensor? gate) -> ()");
  m.def("dit_gelu_tanh(Tensor x) -> Tensor");
  m.def("dit_residual_layer_norm_(Tensor(a!) x, Tensor y, Tensor? gate, Tensor? mul, Tensor? add, bool mul_plus_one, "
        "float eps) -> Tensor");
  m.def("cache_update(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor(a!) states_layer, "
        "Tensor sink_caps_layer, Tensor(b!) committed_vc_layer, Tensor new_k, Tensor new_v, int layer, int t0, "
        "int pass_kind, int shift_pending, int spatial_width, int merge_heads) -> ()");
  m.def("update_descriptors(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, int frames) -> Tensor[]");
  m.def("scatter_copy(Tensor src_ptrs, Tensor lengths, Tensor offsets, Tensor(a!) dst, int col_dim) -> ()");
  m.def("apply_pos_override(Tensor(a!) pos, Tensor starts, Tensor ends, Tensor vals) -> ()");
  m.def("anchor_store_write_frames(Tensor k_seq, Tensor v_seq, Tensor pos_seq, Tensor frame_desc, "
        "Tensor(a!) store_k, Tensor(b!) store_v, Tensor(c!) store_pos) -> ()");
  m.def("refresh_readout_layout(Tensor[] src_k, Tensor[] src_v, Tensor[] src_pos, Tensor(a!) src_ptrs_k, "
        "Tensor(b!) src_ptrs_v, Tensor(c!) src_ptrs_pos, Tensor offsets, Tensor lengths, Tensor flags, "
        "Tensor dynamic_rope_t, Tensor(d!) dst_k_raw, Tensor(e!) dst_v, Tensor(f!) dst_rope_pos, "
        "Tensor(g!) dst_frame_ids, int head_dim, int current_t, str history_time_mapping_mode, "
        "int history_relative_t_max, float history_time_soft_factor) -> ()");
  m.def("pyramidkv_plan(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, int current_t, int pass_kind) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("mega_attend_kv(__torch__.torch.classes.adahead.PyramidKVCacheManager mgr, Tensor states_layer, "
        "int layer_idx, Tensor current_t_list, int sink_mode_code, int sink_clamp_min, int sink_clamp_max, "
        "int decoupled_sink_lag, Tensor freqs_ft_flat, Tensor freqs_fy_flat, Tensor freqs_fx_flat) -> Tensor");
}

TORCH_LIBRARY_IMPL(adahead, CUDA, m) {
  m.impl("pyramidkv_pack", adahead::pyramidkv_pack);
  m.impl("pyramidkv_update", adahead::pyramidkv_update);
  m.impl("mega_state_update", adahead::mega_state_update);
  m.impl("mega_merge_accum", adahead::mega_merge_accum);
  m.impl("mega_merge_accum_weighted", adahead::mega_merge_accum_weighted);
  m.impl("mega_evict_merge", adahead::mega_evict_merge);
  m.impl("ragged_attention", adahead::ragged_attention);
  m.impl("rope_apply", adahead::rope_apply);
  m.impl("dit_layer_norm", adahead::dit_layer_norm);
  m.impl("dit_rms_norm", adahead::dit_rms_norm);
  m.impl("dit_residual_", adahead::dit_residual_);
  m.impl("dit_gelu_tanh", adahead::dit_gelu_tanh);
  m.impl("dit_residual_layer_norm_", adahead::dit_residual_layer_norm_);
  m.impl("cache_update", adahead::cache_update);
  m.impl("scatter_copy", adahead::scatter_copy);
  m.impl("apply_pos_override", adahead::apply_pos_override);
  m.impl("anchor_store_write_frames", adahead::anchor_store_write_frames);
  m.impl("refresh_readout_layout", adahead::refresh_readout_layout);
}

// Ops whose only tensor arguments may live on the host, or that take none,
// dispatch the same implementation whatever the tensor backend.
TORCH_LIBRARY_IMPL(adahead, CompositeExplicitAutograd, m) {
  m.impl("mega_state_perhead_size", adahead::mega_state_perhead_size);
  m.impl("mega_evict_merge_workspace_size", adahead::mega_evict_merge_workspace_size);
  m.impl("ragged_attention_workspace_size", adahead::ragged_attention_workspace_size);
  m.impl("mega_plan", adahead::mega_plan);
  m.impl("mega_plan_multi", adahead::mega_plan_multi);
  m.impl("update_descriptors", adahead::update_descriptors);
  m.impl("mega_attend_kv", adahead::mega_attend_kv);
  m.impl("pyramidkv_plan", adahead::pyramidkv_plan);
}

TORCH_LIBRARY_IMPL(adahead, Meta, m) {
  m.impl("pyramidkv_pack", adahead_meta::pack);
  m.impl("pyramidkv_update", adahead_meta::update);
  m.impl("mega_state_update", adahead_meta::state_update);
  m.impl("mega_merge_accum", adahead_meta::merge);
  m.impl("mega_merge_accum_weighted", adahead_meta::merge_w);
  m.impl("mega_plan", adahead_meta::plan);
  m.impl("mega_plan_multi", adahead_meta::plan_multi);
  m.impl("ragged_attention", adahead_meta::attn);
  m.impl("rope_apply", adahead_meta::rope);
  m.impl("dit_layer_norm", adahead_meta::dit_ln);
  m.impl("dit_rms_norm", adahead_meta::dit_rms);
  m.impl("dit_residual_", adahead_meta::dit_residual);
  m.impl("dit_gelu_tanh", adahead_meta::dit_gelu);
  m.impl("dit_residual_layer_norm_", adahead_meta::dit_res_ln);
  m.impl("cache_update", adahead_meta::cache_update);
  m.impl("scatter_copy", adahead_meta::scatter_copy);
  m.impl("apply_pos_override", adahead_meta::pos_override);
  m.impl("anchor_store_write_frames", adahead_meta::write_frames);
  m.impl("refresh_readout_layout", adahead_meta::refresh);
}
