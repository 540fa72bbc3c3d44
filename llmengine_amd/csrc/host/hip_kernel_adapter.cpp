// hip_kernel_adapter.cpp -- Node -> kernel glue of the HIP backend.
//
// Embedding / Linear / MatMul adapters registered by register_hip_kernels().
// Validation order, error codes and message substrings follow the reference
// device adapters (src/runtime/kernels/cuda_kernel_adapter.cpp:33-108 helpers,
// :110-156 embedding, :158-220 linear, :222-268 matmul); the work runs in the
// gfx950 kernels behind the C ABI of include/mle_q8_0.h.  In addition, every
// buffer's byte size is checked against what the launch will touch, so no
// kernel can read or write outside a bound tensor.
#include <limits>
#include <string>
#include <string_view>

#include "fusion.hpp"
#include "mle_q8_0.h"
#include "minillm_hip/runtime.h"

namespace minillm {

namespace {

Status from_capi(int rc) {
  if (rc == MLE_OK) return Status::make_ok();
  const std::string msg = mle_last_error();
  switch (rc) {
    case MLE_INVALID_ARGUMENT: return Status::invalid_argument(msg);
    case MLE_OUT_OF_RANGE: return Status::out_of_range(msg);
    case MLE_SHAPE_MISMATCH: return Status::shape_mismatch(msg);
    case MLE_UNSUPPORTED: return Status::unsupported(msg);
    default: return Status::runtime_error(msg);
  }
}

expected<Tensor*, Status> get_tensor(ValueId id, RuntimeContext& ctx, std::string_view role) {
  Tensor* t = ctx.get(id);
  if (!t)
    return unexpected(Status::runtime_error(std::string(role) + " tensor not found for ValueId %" +
                                            std::to_string(id.value)));
  return t;
}

Status check_allocated(const Tensor* t, std::string_view name) {
  if (!t->is_allocated()) return Status::runtime_error(std::string(name) + " tensor not allocated");
  return Status::make_ok();
}

Status check_hip_device(const Tensor* t, std::string_view name) {
  if (t->device().type != DeviceType::HIP)
    return Status::unsupported(std::string(name) + " must be a HIP tensor, got " +
                               t->device().to_string());
  return Status::make_ok();
}

// Linear bias: Float32 or BFloat16, as the reference's CUDA adapter accepts
// (cuda_kernel_adapter.cpp:48-59, 204-218).
Status check_hip_float_or_bf16(const Tensor* t, std::string_view name) {
  TRY(check_allocated(t, name));
  TRY(check_hip_device(t, name));
  if (t->dtype() == DType::Float32 || t->dtype() == DType::BFloat16) return Status::make_ok();
  return Status::unsupported(std::string(name) + " supports Float32 or BFloat16, got " +
                             std::string(dtype_name(t->dtype())));
}

Status check_hip_float(const Tensor* t, std::string_view name) {
  TRY(check_allocated(t, name));
  TRY(check_hip_device(t, name));
  if (t->dtype() != DType::Float32)
    return Status::unsupported(std::string(name) + " only supports Float32, got " +
                               std::string(dtype_name(t->dtype())));
  return Status::make_ok();
}

// The HIP backend implements the Q8_0 weight path only.
Status check_hip_q8_weight(const Tensor* t, std::string_view name) {
  TRY(check_allocated(t, name));
  TRY(check_hip_device(t, name));
  if (t->dtype() != DType::Q8_0)
    return Status::unsupported(std::string(name) +
                               " supports Q8_0 weights on the HIP backend, got " +
                               std::string(dtype_name(t->dtype())));
  return Status::make_ok();
}

Status check_q8_block_aligned(int64_t block_dim, std::string_view op) {
  if (block_dim % static_cast<int64_t>(kQ8_0BlockElems) == 0) return Status::make_ok();
  return Status::unsupported(std::string(op) +
                             " Q8_0 weights require the packed dimension to be a multiple of 32, got " +
                             std::to_string(block_dim));
}

Status check_q8_storage_bytes(const Tensor* t, std::string_view name) {
  auto n = t->numel();
  if (!n) return n.error();
  const size_t need = q8_0_bytes(*n);
  if (t->allocated_bytes() < need)
    return Status::out_of_range(std::string(name) + " Q8_0 raw storage is too small: need " +
                                std::to_string(need) + " bytes, got " +
                                std::to_string(t->allocated_bytes()));
  return Status::make_ok();
}

// MatMul reads GGUF blocks along N; a weight re-tiled in place by
// HipExecutor::tile_weights(ctx, true) holds 16-row tiles along K.
Status check_raw_layout(const Tensor* t, std::string_view name) {
  if (t->storage_layout() == StorageLayout::Raw) return Status::make_ok();
  return Status::unsupported(std::string(name) +
                             " holds Q8_0 16-row tiles (re-tiled in place); this op reads raw "
                             "Q8_0 blocks");
}

// Storage of a Q8_0 weight in its layout: raw blocks, or N x K in 16-row tiles.
Status check_q8_layout_bytes(const Tensor* t, int N, int K, std::string_view name) {
  if (t->storage_layout() == StorageLayout::Raw) return check_q8_storage_bytes(t, name);
  const size_t need = hip::q8_0_tiled_bytes(N, K);
  if (t->allocated_bytes() < need)
    return Status::out_of_range(std::string(name) + " Q8_0 tiled storage is too small: need " +
                                std::to_string(need) + " bytes, got " +
                                std::to_string(t->allocated_bytes()));
  return Status::make_ok();
}

Status check_storage_bytes(const Tensor* t, size_t need, std::string_view name) {
  if (t->allocated_bytes() < need)
    return Status::out_of_range(std::string(name) + " storage is too small: need " +
                                std::to_string(need) + " bytes, got " +
                                std::to_string(t->allocated_bytes()));
  return Status::make_ok();
}

expected<int, Status> checked_dim(int64_t v, std::string_view role) {
  if (v < 0 || v > std::numeric_limits<int>::max())
    return unexpected(Status::unsupported(std::string(role) + " dimension is outside int range"));
  return static_cast<int>(v);
}

expected<int, Status> checked_count(size_t v, std::string_view role) {
  if (v > static_cast<size_t>(std::numeric_limits<int>::max()))
    return unexpected(Status::unsupported(std::string(role) + " is too large for int indexing"));
  return static_cast<int>(v);
}

Status kernel_embedding(const Node& node, RuntimeContext& ctx) {
  if (node.inputs().size() < 2 || node.outputs().empty())
    return Status::invalid_argument("Embedding expects inputs [input_ids, weight] and one output");
  auto ids = get_tensor(node.inputs()[0], ctx, "input_ids");
  if (!ids) return ids.error();
  auto wt = get_tensor(node.inputs()[1], ctx, "weight");
  if (!wt) return wt.error();
  auto ot = get_tensor(node.outputs()[0], ctx, "output");
  if (!ot) return ot.error();

  TRY(check_allocated(*ids, "input_ids"));
  TRY(check_hip_device(*ids, "input_ids"));
  if ((*ids)->dtype() != DType::Int32)
    return Status::unsupported("input_ids only supports Int32, got " +
                               std::string(dtype_name((*ids)->dtype())));
  TRY(check_hip_q8_weight(*wt, "weight"));
  TRY(check_hip_float(*ot, "output"));
  if ((*wt)->shape().rank() != 2) return Status::shape_mismatch("Embedding weight must be rank 2");

  auto n_ids = (*ids)->numel();
  if (!n_ids) return n_ids.error();
  auto seq_len = checked_count(*n_ids, "embedding input_ids");
  if (!seq_len) return seq_len.error();
  auto vocab = checked_dim((*wt)->shape().dim(0), "embedding vocab");
  if (!vocab) return vocab.error();
  auto hidden = checked_dim((*wt)->shape().dim(1), "embedding hidden");
  if (!hidden) return hidden.error();
  TRY(check_q8_block_aligned(*hidden, "embedding"));
  TRY(check_q8_layout_bytes(*wt, *vocab, *hidden, "embedding weight"));
  TRY(check_storage_bytes(*ids, static_cast<size_t>(*seq_len) * 4, "input_ids"));
  TRY(check_storage_bytes(*ot, static_cast<size_t>(*seq_len) * static_cast<size_t>(*hidden) * 4,
                          "output"));
  if ((*wt)->storage_layout() == StorageLayout::Q8_0Tiled)
    return hip::embedding_tiled(static_cast<const uint8_t*>((*wt)->data()),
                                static_cast<const int*>((*ids)->data()),
                                static_cast<float*>((*ot)->data()), *seq_len, *vocab, *hidden,
                                ctx.hip_stream());
  return hip::embedding(static_cast<const uint8_t*>((*wt)->data()),
                        static_cast<const int*>((*ids)->data()),
                        static_cast<float*>((*ot)->data()), *seq_len, *vocab, *hidden,
                        ctx.hip_stream());
}

Status kernel_linear(const Node& node, RuntimeContext& ctx) {
  if (node.inputs().size() < 2 || node.outputs().empty())
    return Status::invalid_argument("Linear expects inputs [x, weight, (bias)] and one output");
  auto xt = get_tensor(node.inputs()[0], ctx, "x");
  if (!xt) return xt.error();
  auto wt = get_tensor(node.inputs()[1], ctx, "weight");
  if (!wt) return wt.error();
  auto ot = get_tensor(node.outputs()[0], ctx, "output");
  if (!ot) return ot.error();

  TRY(check_hip_float(*xt, "x"));
  TRY(check_hip_q8_weight(*wt, "weight"));
  TRY(check_hip_float(*ot, "output"));
  if ((*wt)->shape().rank() != 2) return Status::shape_mismatch("Linear weight must be rank 2");
  if ((*xt)->shape().rank() == 0) return Status::shape_mismatch("linear x expects rank >= 1");

  size_t rows = 1;
  for (size_t i = 0; i + 1 < (*xt)->shape().rank(); ++i)
    rows *= static_cast<size_t>((*xt)->shape().dim(i));
  auto M = checked_count(rows, "linear x");
  if (!M) return M.error();
  auto K = checked_dim((*xt)->shape().dim((*xt)->shape().rank() - 1), "linear x");
  if (!K) return K.error();
  auto N = checked_dim((*wt)->shape().dim(0), "linear output");
  if (!N) return N.error();
  auto wk = checked_dim((*wt)->shape().dim(1), "linear weight input");
  if (!wk) return wk.error();
  if (*wk != *K)
    return Status::shape_mismatch("Linear x last dimension must match weight input dimension");

  const void* bias = nullptr;
  bool bias_bf16 = false;
  if (node.inputs().size() >= 3) {
    auto bt = get_tensor(node.inputs()[2], ctx, "bias");
    if (!bt) return bt.error();
    TRY(check_hip_float_or_bf16(*bt, "bias"));
    if ((*bt)->shape().rank() != 1 || (*bt)->shape().dim(0) != *N)
      return Status::shape_mismatch("Linear bias shape must match output features");
    bias_bf16 = (*bt)->dtype() == DType::BFloat16;
    TRY(check_storage_bytes(*bt, static_cast<size_t>(*N) * (bias_bf16 ? 2 : 4), "bias"));
    bias = (*bt)->data();
  }
  TRY(check_q8_block_aligned(*K, "linear"));
  TRY(check_q8_layout_bytes(*wt, *N, *K, "linear weight"));
  TRY(check_storage_bytes(*xt, static_cast<size_t>(*M) * static_cast<size_t>(*K) * 4, "x"));
  TRY(check_storage_bytes(*ot, static_cast<size_t>(*M) * static_cast<size_t>(*N) * 4, "output"));
  if ((*wt)->storage_layout() == StorageLayout::Q8_0Tiled) {
    const auto* x = static_cast<const float*>((*xt)->data());
    const auto* w = static_cast<const uint8_t*>((*wt)->data());
    auto* y = static_cast<float*>((*ot)->data());
    return bias_bf16 ? hip::sgemm_nt_tiled_bias_bf16(x, w, y, *M, *N, *K,
                                                     static_cast<const uint16_t*>(bias),
                                                     ctx.hip_stream())
                     : hip::sgemm_nt_tiled(x, w, y, *M, *N, *K, static_cast<const float*>(bias),
                                           ctx.hip_stream());
  }
  if (bias_bf16)
    return hip::sgemm_nt_bias_bf16(static_cast<const float*>((*xt)->data()),
                                   static_cast<const uint8_t*>((*wt)->data()),
                                   static_cast<float*>((*ot)->data()), *M, *N, *K,
                                   static_cast<const uint16_t*>(bias), ctx.hip_stream());
  return hip::sgemm_nt(static_cast<const float*>((*xt)->data()),
                       static_cast<const uint8_t*>((*wt)->data()),
                       static_cast<float*>((*ot)->data()), *M, *N, *K,
                       static_cast<const float*>(bias), ctx.hip_stream());
}

Status kernel_swiglu(const Node& node, RuntimeContext& ctx) {
  if (node.inputs().size() < 2 || node.outputs().empty())
    return Status::invalid_argument("SwiGLU expects inputs [gate, up] and one output");
  auto gt = get_tensor(node.inputs()[0], ctx, "gate");
  if (!gt) return gt.error();
  auto ut = get_tensor(node.inputs()[1], ctx, "up");
  if (!ut) return ut.error();
  auto ot = get_tensor(node.outputs()[0], ctx, "output");
  if (!ot) return ot.error();
  TRY(check_hip_float(*gt, "gate"));
  TRY(check_hip_float(*ut, "up"));
  TRY(check_hip_float(*ot, "output"));
  auto n = (*ot)->numel();
  if (!n) return n.error();
  TRY(check_storage_bytes(*gt, *n * 4, "gate"));
  TRY(check_storage_bytes(*ut, *n * 4, "up"));
  TRY(check_storage_bytes(*ot, *n * 4, "output"));
  return from_capi(mle_swiglu_f32(static_cast<const float*>((*gt)->data()),
                                  static_cast<const float*>((*ut)->data()),
                                  static_cast<float*>((*ot)->data()), (int64_t)*n,
                                  ctx.hip_stream()));
}

// Operands of one Q8_0 Linear node, validated as kernel_linear validates them.
struct LinearOperands {
  const float* x = nullptr;
  const uint8_t* w = nullptr;
  bool w_tiled = false;  // w holds 16-row tiles (re-tiled in place), not GGUF blocks
  const void* bias = nullptr;
  bool bias_bf16 = false;
  float* y = nullptr;
  int M = 0, N = 0, K = 0;
  ValueId x_id;
};

expected<LinearOperands, Status> linear_operands(const Node& node, RuntimeContext& ctx) {
  if (node.op_type() != OpType::Linear || node.inputs().size() < 2 || node.outputs().empty())
    return unexpected(Status::invalid_argument("not a Linear node"));
  auto xt = get_tensor(node.inputs()[0], ctx, "x");
  if (!xt) return unexpected(xt.error());
  auto wt = get_tensor(node.inputs()[1], ctx, "weight");
  if (!wt) return unexpected(wt.error());
  auto ot = get_tensor(node.outputs()[0], ctx, "output");
  if (!ot) return unexpected(ot.error());
  Status st = check_hip_float(*xt, "x");
  if (st.ok()) st = check_hip_q8_weight(*wt, "weight");
  if (st.ok()) st = check_hip_float(*ot, "output");
  if (!st.ok()) return unexpected(st);
  if ((*wt)->shape().rank() != 2 || (*xt)->shape().rank() == 0)
    return unexpected(Status::shape_mismatch("Linear operand ranks"));
  size_t rows = 1;
  for (size_t i = 0; i + 1 < (*xt)->shape().rank(); ++i)
    rows *= static_cast<size_t>((*xt)->shape().dim(i));
  auto M = checked_count(rows, "linear x");
  auto K = checked_dim((*xt)->shape().dim((*xt)->shape().rank() - 1), "linear x");
  auto N = checked_dim((*wt)->shape().dim(0), "linear output");
  auto wk = checked_dim((*wt)->shape().dim(1), "linear weight input");
  if (!M || !K || !N || !wk || *wk != *K)
    return unexpected(Status::shape_mismatch("Linear operand shapes"));
  LinearOperands o;
  if (node.inputs().size() >= 3) {
    auto bt = get_tensor(node.inputs()[2], ctx, "bias");
    if (!bt) return unexpected(bt.error());
    st = check_hip_float_or_bf16(*bt, "bias");
    if (!st.ok()) return unexpected(st);
    if ((*bt)->shape().rank() != 1 || (*bt)->shape().dim(0) != *N)
      return unexpected(Status::shape_mismatch("Linear bias shape must match output features"));
    o.bias_bf16 = (*bt)->dtype() == DType::BFloat16;
    st = check_storage_bytes(*bt, static_cast<size_t>(*N) * (o.bias_bf16 ? 2 : 4), "bias");
    if (!st.ok()) return unexpected(st);
    o.bias = (*bt)->data();
  }
  st = check_q8_block_aligned(*K, "linear");
  if (st.ok()) st = check_q8_layout_bytes(*wt, *N, *K, "linear weight");
  if (st.ok())
    st = check_storage_bytes(*xt, static_cast<size_t>(*M) * static_cast<size_t>(*K) * 4, "x");
  if (st.ok())
    st = check_storage_bytes(*ot, static_cast<size_t>(*M) * static_cast<size_t>(*N) * 4,
                             "output");
  if (!st.ok()) return unexpected(st);
  o.x = static_cast<const float*>((*xt)->data());
  o.w = static_cast<const uint8_t*>((*wt)->data());
  o.w_tiled = (*wt)->storage_layout() == StorageLayout::Q8_0Tiled;
  o.y = static_cast<float*>((*ot)->data());
  o.M = *M;
  o.N = *N;
  o.K = *K;
  o.x_id = node.inputs()[0];
  return o;
}

Status kernel_matmul(const Node& node, RuntimeContext& ctx) {
  if (node.inputs().size() < 2 || node.outputs().empty())
    return Status::invalid_argument("MatMul expects inputs [a, b] and one output");
  auto at = get_tensor(node.inputs()[0], ctx, "a");
  if (!at) return at.error();
  auto bt = get_tensor(node.inputs()[1], ctx, "b");
  if (!bt) return bt.error();
  auto ot = get_tensor(node.outputs()[0], ctx, "output");
  if (!ot) return ot.error();

  TRY(check_hip_float(*at, "a"));
  TRY(check_hip_q8_weight(*bt, "b"));
  TRY(check_hip_float(*ot, "output"));
  if ((*at)->shape().rank() != 2 || (*bt)->shape().rank() != 2)
    return Status::shape_mismatch("HIP MatMul currently expects rank-2 tensors");
  auto M = checked_dim((*at)->shape().dim(0), "matmul M");
  if (!M) return M.error();
  auto K = checked_dim((*at)->shape().dim(1), "matmul K");
  if (!K) return K.error();
  auto bk = checked_dim((*bt)->shape().dim(0), "matmul B K");
  if (!bk) return bk.error();
  auto N = checked_dim((*bt)->shape().dim(1), "matmul N");
  if (!N) return N.error();
  if (*bk != *K) return Status::shape_mismatch("MatMul inner dimensions differ");
  TRY(check_q8_block_aligned(*K, "matmul reduction dimension"));
  TRY(check_q8_block_aligned(*N, "matmul output dimension"));
  TRY(check_raw_layout(*bt, "matmul b"));
  TRY(check_q8_storage_bytes(*bt, "matmul b"));
  TRY(check_storage_bytes(*at, static_cast<size_t>(*M) * static_cast<size_t>(*K) * 4, "a"));
  TRY(check_storage_bytes(*ot, static_cast<size_t>(*M) * static_cast<size_t>(*N) * 4, "output"));
  return hip::sgemm(static_cast<const float*>((*at)->data()),
                    static_cast<const uint8_t*>((*bt)->data()),
                    static_cast<float*>((*ot)->data()), *M, *N, *K, ctx.hip_stream());
}

}  // namespace

namespace hip {

Status sgemm_nt(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
                const float* bias, hipStream_t stream) {
  return from_capi(mle_q8_0_linear(A, B_q8_0, bias, C, M, N, K, stream));
}

Status sgemm_nt_bias_bf16(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
                          const uint16_t* bias_bf16, hipStream_t stream) {
  return from_capi(mle_q8_0_linear_bias_bf16(A, B_q8_0, bias_bf16, C, M, N, K, stream));
}

Status sgemm_nt_tiled_bias_bf16(const float* A, const uint8_t* B_tiled, float* C, int M, int N,
                                int K, const uint16_t* bias_bf16, hipStream_t stream) {
  return from_capi(mle_q8_0_linear_tiled_bias_bf16(A, B_tiled, bias_bf16, C, M, N, K, stream));
}

Status sgemm(const float* A, const uint8_t* B_q8_0, float* C, int M, int N, int K,
             hipStream_t stream) {
  return from_capi(mle_q8_0_matmul(A, B_q8_0, C, M, N, K, stream));
}

Status embedding(const uint8_t* weight_q8_0, const int* ids, float* out, int seq_len,
                 int vocab_size, int hidden, hipStream_t stream) {
  return from_capi(mle_q8_0_embedding(weight_q8_0, reinterpret_cast<const int32_t*>(ids), out,
                                      seq_len, vocab_size, hidden, stream));
}

Status embedding_tiled(const uint8_t* weight_tiled, const int* ids, float* out, int seq_len,
                       int vocab_size, int hidden, hipStream_t stream) {
  return from_capi(mle_q8_0_embedding_tiled(weight_tiled, reinterpret_cast<const int32_t*>(ids),
                                            out, seq_len, vocab_size, hidden, stream));
}

Status dequantize_q8_0(const uint8_t* src_q8_0, float* out, int64_t n, hipStream_t stream) {
  return from_capi(mle_q8_0_dequantize(src_q8_0, out, n, stream));
}

Status linear_swiglu(const float* x, const uint8_t* w_gate_q8_0, const uint8_t* w_up_q8_0,
                     float* y, int M, int N, int K, hipStream_t stream) {
  return from_capi(mle_q8_0_linear_swiglu(x, w_gate_q8_0, w_up_q8_0, y, M, N, K, stream));
}

Status linear_multi(const float* x, int count, const uint8_t* const* w_q8_0,
                    const float* const* bias, float* const* y, const int* N, int M, int K,
                    hipStream_t stream) {
  return from_capi(mle_q8_0_linear_multi(x, count, w_q8_0, bias, y, N, M, K, stream));
}

Status argmax(const float* logits, int rows, int n, int32_t* idx, float* val,
              hipStream_t stream) {
  return from_capi(mle_argmax_f32(logits, rows, n, idx, val, stream));
}

Status top_tokens(const float* logits, int rows, int n, int top_n, float temperature,
                  int32_t* ids, float* probs, hipStream_t stream) {
  return from_capi(mle_top_tokens_f32(logits, rows, n, top_n, temperature, ids, probs, stream));
}

size_t q8_0_tiled_bytes(int N, int K) { return mle_q8_0_tiled_bytes(N, K); }

Status tile_q8_0(const uint8_t* w_q8_0, uint8_t* w_tiled, int N, int K, hipStream_t stream) {
  return from_capi(mle_q8_0_tile(w_q8_0, w_tiled, N, K, stream));
}

Status sgemm_nt_tiled(const float* A, const uint8_t* B_tiled, float* C, int M, int N, int K,
                      const float* bias, hipStream_t stream) {
  return from_capi(mle_q8_0_linear_tiled(A, B_tiled, bias, C, M, N, K, stream));
}

Status linear_swiglu_tiled(const float* x, const uint8_t* w_gate_tiled,
                           const uint8_t* w_up_tiled, float* y, int M, int N, int K,
                           hipStream_t stream) {
  return from_capi(
      mle_q8_0_linear_swiglu_tiled(x, w_gate_tiled, w_up_tiled, y, M, N, K, stream));
}

Status linear_multi_tiled(const float* x, int count, const uint8_t* const* w_tiled,
                          const float* const* bias, float* const* y, const int* N, int M,
                          int K, hipStream_t stream) {
  return from_capi(mle_q8_0_linear_multi_tiled(x, count, w_tiled, bias, y, N, M, K, stream));
}

}  // namespace hip

namespace detail {

const uint8_t* tiled_copy_of(const TiledWeights* tiled, const void* raw, int64_t N, int64_t K) {
  if (tiled == nullptr) return nullptr;
  auto it = tiled->find(raw);
  if (it == tiled->end() || it->second.N != N || it->second.K != K) return nullptr;
  return it->second.data;
}

expected<bool, Status> run_tiled_linear(const Node& node, RuntimeContext& ctx,
                                        const TiledWeights* tiled) {
  auto o = linear_operands(node, ctx);
  if (!o) return false;
  const uint8_t* t = o->w_tiled ? o->w : tiled_copy_of(tiled, o->w, o->N, o->K);
  if (t == nullptr) return false;
  const Status st =
      o->bias_bf16
          ? hip::sgemm_nt_tiled_bias_bf16(o->x, t, o->y, o->M, o->N, o->K,
                                          static_cast<const uint16_t*>(o->bias), ctx.hip_stream())
          : hip::sgemm_nt_tiled(o->x, t, o->y, o->M, o->N, o->K,
                                static_cast<const float*>(o->bias), ctx.hip_stream());
  if (!st.ok()) return unexpected(st);
  return true;
}

expected<bool, Status> run_fused_swiglu(const Node& gate, const Node& up, const Node& sw,
                                        RuntimeContext& ctx, const TiledWeights* tiled,
                                        bool* used_tiled) {
  auto g = linear_operands(gate, ctx);
  auto u = linear_operands(up, ctx);
  if (!g || !u || g->bias || u->bias || g->x != u->x || g->M != u->M || g->N != u->N ||
      g->K != u->K || sw.outputs().empty())
    return false;
  Tensor* ot = ctx.get(sw.outputs()[0]);
  if (!ot || !check_hip_float(ot, "output").ok() ||
      !check_storage_bytes(ot, static_cast<size_t>(g->M) * g->N * 4, "output").ok())
    return false;
  const uint8_t* tg = g->w_tiled ? g->w : tiled_copy_of(tiled, g->w, g->N, g->K);
  const uint8_t* tu = u->w_tiled ? u->w : tiled_copy_of(tiled, u->w, u->N, u->K);
  // One weight re-tiled in place and the other raw with no copy: node by node.
  if ((g->w_tiled || u->w_tiled) && !(tg && tu)) return false;
  if (used_tiled) *used_tiled = tg && tu;
  const Status st =
      tg && tu ? hip::linear_swiglu_tiled(g->x, tg, tu, static_cast<float*>(ot->data()), g->M,
                                          g->N, g->K, ctx.hip_stream())
               : hip::linear_swiglu(g->x, g->w, u->w, static_cast<float*>(ot->data()), g->M,
                                    g->N, g->K, ctx.hip_stream());
  if (!st.ok()) return unexpected(st);
  return true;
}

expected<bool, Status> run_fused_multi(const std::vector<const Node*>& nodes,
                                       RuntimeContext& ctx, const TiledWeights* tiled,
                                       bool* used_tiled) {
  if (nodes.size() < 2 || nodes.size() > 3) return false;
  const uint8_t* w[3];
  bool in_place[3] = {false, false, false};
  const float* b[3];
  float* y[3];
  int N[3];
  LinearOperands first;
  for (size_t i = 0; i < nodes.size(); ++i) {
    auto o = linear_operands(*nodes[i], ctx);
    if (!o || o->bias_bf16) return false;  // BF16 biases run node by node
    if (i == 0) first = *o;
    else if (o->x != first.x || o->M != first.M || o->K != first.K) return false;
    w[i] = o->w;
    in_place[i] = o->w_tiled;
    b[i] = static_cast<const float*>(o->bias);
    y[i] = o->y;
    N[i] = o->N;
  }
  const uint8_t* tw[3] = {nullptr, nullptr, nullptr};
  bool all_tiled = true, any_in_place = false;
  for (size_t i = 0; i < nodes.size(); ++i) {
    tw[i] = in_place[i] ? w[i] : tiled_copy_of(tiled, w[i], N[i], first.K);
    all_tiled = all_tiled && tw[i] != nullptr;
    any_in_place = any_in_place || in_place[i];
  }
  if (any_in_place && !all_tiled) return false;  // mixed layouts: node by node
  if (used_tiled) *used_tiled = all_tiled;
  const Status st =
      all_tiled ? hip::linear_multi_tiled(first.x, static_cast<int>(nodes.size()), tw, b, y, N,
                                          first.M, first.K, ctx.hip_stream())
                : hip::linear_multi(first.x, static_cast<int>(nodes.size()), w, b, y, N,
                                    first.M, first.K, ctx.hip_stream());
  if (!st.ok()) return unexpected(st);
  return true;
}

}  // namespace detail

void register_hip_kernels(KernelRegistry& registry) {
  registry.register_kernel(DeviceType::HIP, OpType::Embedding, kernel_embedding);
  registry.register_kernel(DeviceType::HIP, OpType::Linear, kernel_linear);
  registry.register_kernel(DeviceType::HIP, OpType::MatMul, kernel_matmul);
  registry.register_kernel(DeviceType::HIP, OpType::SwiGLU, kernel_swiglu);
}

}  // namespace minillm
