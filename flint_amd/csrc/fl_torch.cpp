// Torch-extension binding of the C ABI (pybind11 over torch tensors), the form in which the
// reference exposes its kernels: decode_mega_launch / verify_mega_launch are pybind ops over
// torch tensors (reference kernels/megakernel_decode.cu:204-250, kernels/verify_mega.cu:246-298).
// A thin layer: it checks dtype, device, contiguity and shape (TORCH_CHECK, which the reference
// leaves out), allocates the outputs through torch's caching allocator as the reference does,
// and calls the C ABI on the stream handle the caller passes. The state the C ABI keeps between
// calls (exchange buffers, the bound KV cache) lives in an Engine object, which holds references
// to every tensor it points into, so none can be freed under it.
#include <torch/extension.h>

#include <vector>

#include "../../include/flint_amd.h"

namespace {

void check_dev(const torch::Tensor& t, torch::ScalarType dt, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, ": a device tensor is required");
  TORCH_CHECK(t.scalar_type() == dt, name, ": dtype ", t.scalar_type(), ", expected ", dt);
  TORCH_CHECK(t.is_contiguous(), name, ": must be contiguous");
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == FL_OK, what, " failed with status ", rc,
              rc == FL_E_ARG ? " (FL_E_ARG: bad argument / shape)"
              : rc == FL_E_POS ? " (FL_E_POS: position beyond the cache or rope table)"
              : rc == FL_E_M ? " (FL_E_M: verify width out of range)"
              : rc == FL_E_LAUNCH ? " (FL_E_LAUNCH)"
              : rc == FL_E_TIMEOUT ? " (FL_E_TIMEOUT)" : "");
}

void* stream_of(int64_t s) { return reinterpret_cast<void*>(static_cast<intptr_t>(s)); }

class Engine {
 public:
  // Weights in this library's packed layout (flint_amd.model.PackedModel's tensors), the bf16 KV
  // cache [NL, NKV, S, 64] (caller-owned, as chat.py:68-69) and the ModelArgs scalars.
  Engine(torch::Tensor wqkv_q, torch::Tensor wqkv_sz, torch::Tensor wo_q, torch::Tensor wo_sz,
         torch::Tensor wgu_q, torch::Tensor wgu_sz, torch::Tensor wd_q, torch::Tensor wd_sz,
         torch::Tensor attn_norm, torch::Tensor ffn_norm, torch::Tensor final_norm, torch::Tensor embed,
         torch::Tensor rope, torch::Tensor k_cache, torch::Tensor v_cache, double norm_eps,
         double emb_mult, double attn_scale, double resid_mult, double logits_scaling) {
    for (auto* t : {&wqkv_q, &wqkv_sz, &wo_q, &wo_sz, &wgu_q, &wgu_sz, &wd_q, &wd_sz})
      check_dev(*t, torch::kInt32, "packed int4 weights");
    for (auto* t : {&attn_norm, &ffn_norm, &final_norm, &embed, &rope, &k_cache, &v_cache})
      check_dev(*t, torch::kBFloat16, "bf16 weights / cache");
    TORCH_CHECK(k_cache.dim() == 4 && k_cache.size(3) == FL_HEAD_DIM && v_cache.sizes() == k_cache.sizes(),
                "k_cache / v_cache: [NL, NKV, S, 64]");
    TORCH_CHECK(embed.dim() == 2 && wqkv_q.dim() == 3 && wgu_q.dim() == 3 && rope.dim() == 3,
                "embed [V, D], packed weights [NL, N, K / 8], rope [L, 32, 2]");
    d_.n_layer = (int32_t)k_cache.size(0);
    d_.n_kv_head = (int32_t)k_cache.size(1);
    d_.dim = (int32_t)embed.size(1);
    d_.vocab = (int32_t)embed.size(0);
    d_.inter = (int32_t)(wgu_q.size(1) / 2);
    d_.n_head = (int32_t)(wqkv_q.size(1) / FL_HEAD_DIM) - 2 * d_.n_kv_head;
    d_.norm_eps = (float)norm_eps;
    d_.emb_mult = (float)emb_mult;
    d_.attn_scale = (float)attn_scale;
    d_.resid_mult = (float)resid_mult;
    d_.logits_scaling = (float)logits_scaling;
    TORCH_CHECK(wqkv_q.size(0) == d_.n_layer && wqkv_q.size(2) * 8 == d_.dim, "wqkv_q: [NL, (NH + 2 NKV) 64, D / 8]");
    keep_ = {wqkv_q, wqkv_sz, wo_q, wo_sz, wgu_q, wgu_sz, wd_q, wd_sz, attn_norm, ffn_norm, final_norm,
             embed, rope, k_cache, v_cache};
    w_.wqkv_q = reinterpret_cast<const uint32_t*>(wqkv_q.data_ptr());
    w_.wqkv_sz = reinterpret_cast<const uint32_t*>(wqkv_sz.data_ptr());
    w_.wo_q = reinterpret_cast<const uint32_t*>(wo_q.data_ptr());
    w_.wo_sz = reinterpret_cast<const uint32_t*>(wo_sz.data_ptr());
    w_.wgu_q = reinterpret_cast<const uint32_t*>(wgu_q.data_ptr());
    w_.wgu_sz = reinterpret_cast<const uint32_t*>(wgu_sz.data_ptr());
    w_.wd_q = reinterpret_cast<const uint32_t*>(wd_q.data_ptr());
    w_.wd_sz = reinterpret_cast<const uint32_t*>(wd_sz.data_ptr());
    w_.attn_norm = reinterpret_cast<const uint16_t*>(attn_norm.data_ptr());
    w_.ffn_norm = reinterpret_cast<const uint16_t*>(ffn_norm.data_ptr());
    w_.final_norm = reinterpret_cast<const uint16_t*>(final_norm.data_ptr());
    w_.embed = reinterpret_cast<const uint16_t*>(embed.data_ptr());
    w_.rope = reinterpret_cast<const uint16_t*>(rope.data_ptr());
    w_.rope_len = (int32_t)rope.size(0);
    // the tiled copies the verify kernel reads (fl_tile_int4), made once here on the default
    // stream and kept with the other tensors
    auto tile = [&](const torch::Tensor& q) {
      torch::Tensor t = torch::empty_like(q);
      check_rc(fl_tile_int4(reinterpret_cast<const uint32_t*>(q.data_ptr()), reinterpret_cast<uint32_t*>(t.data_ptr()),
                            (int32_t)(q.numel() / q.size(-1)), (int32_t)(q.size(-1) * 8), nullptr),
               "fl_tile_int4");
      keep_.push_back(t);
      return reinterpret_cast<const uint32_t*>(t.data_ptr());
    };
    w_.wqkv_t = tile(wqkv_q);
    w_.wo_t = tile(wo_q);
    w_.wgu_t = tile(wgu_q);
    w_.wd_t = tile(wd_q);
    check_rc(fl_state_create(&d_, (int32_t)k_cache.size(2), reinterpret_cast<uint16_t*>(k_cache.data_ptr()),
                             reinterpret_cast<uint16_t*>(v_cache.data_ptr()), &st_),
             "fl_state_create");
  }
  ~Engine() {
    if (st_) fl_state_destroy(st_);
  }
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  // decode_mega_launch(..., h, kc, vc, pos, ...) -> logits (reference megakernel_decode.cu:204-237):
  // h (bf16 [D]) is the layer-0 input and receives the final residual in place.
  torch::Tensor decode_hidden(torch::Tensor h, int64_t pos, int64_t stream) {
    check_dev(h, torch::kBFloat16, "h");
    TORCH_CHECK(h.numel() == d_.dim, "h: [", d_.dim, "]");
    auto logits = torch::empty({d_.vocab}, h.options().dtype(torch::kFloat32));
    check_rc(fl_decode_hidden(&w_, st_, reinterpret_cast<uint16_t*>(h.data_ptr()), (int32_t)pos, nullptr,
                              logits.data_ptr<float>(), nullptr, stream_of(stream)),
             "fl_decode_hidden");
    return logits;
  }

  // one greedy decode step from a token id (device int32 [1]): (argmax token [1], logits [V])
  std::tuple<torch::Tensor, torch::Tensor> decode_step(torch::Tensor token, int64_t pos, int64_t stream) {
    check_dev(token, torch::kInt32, "token");
    TORCH_CHECK(token.numel() == 1, "token: one id");
    auto out = torch::empty({1}, token.options());
    auto logits = torch::empty({d_.vocab}, token.options().dtype(torch::kFloat32));
    check_rc(fl_decode_step(&w_, st_, token.data_ptr<int32_t>(), (int32_t)pos, out.data_ptr<int32_t>(),
                            logits.data_ptr<float>(), nullptr, stream_of(stream)),
             "fl_decode_step");
    return {out, logits};
  }

  // verify_mega_launch(..., h[M], kc, vc, depth, amask, pos, M) -> [logits [M, V], feat [M, D]]
  // (reference verify_mega.cu:246-283), from token ids; plus the per-token argmax [M].
  std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> verify(torch::Tensor tokens, torch::Tensor depth,
                                                                 torch::Tensor amask, int64_t pos,
                                                                 int64_t stream) {
    check_dev(tokens, torch::kInt32, "tokens");
    check_dev(depth, torch::kInt32, "depth");
    check_dev(amask, torch::kUInt8, "amask");
    const int64_t m = tokens.numel();
    TORCH_CHECK(m >= 1 && m <= FL_MAX_VERIFY, "tokens: 1..", FL_MAX_VERIFY, " ids");
    TORCH_CHECK(depth.numel() == m && amask.numel() == m * m, "depth [M], amask [M, M]");
    auto out = torch::empty({m}, tokens.options());
    auto logits = torch::empty({m, d_.vocab}, tokens.options().dtype(torch::kFloat32));
    auto feat = torch::empty({m, d_.dim}, tokens.options().dtype(torch::kBFloat16));
    check_rc(fl_verify(&w_, st_, tokens.data_ptr<int32_t>(), (int32_t)m, depth.data_ptr<int32_t>(),
                       amask.data_ptr<uint8_t>(), (int32_t)pos, out.data_ptr<int32_t>(), logits.data_ptr<float>(),
                       reinterpret_cast<uint16_t*>(feat.data_ptr()), stream_of(stream)),
             "fl_verify");
    return {out, logits, feat};
  }

  // raise if a launch recorded an error (synchronises the stream)
  void check(int64_t stream) { check_rc(fl_state_check(st_, stream_of(stream)), "fl_state_check"); }

 private:
  fl_model_desc d_{};
  fl_weights w_{};
  fl_state* st_ = nullptr;
  std::vector<torch::Tensor> keep_;
};

// WeightOnlyInt4Linear.forward (reference engine/quantize.py:517-525): y = x . dq^T, M <= 32 rows
torch::Tensor int4_linear(torch::Tensor x, torch::Tensor q, torch::Tensor sz, int64_t stream) {
  check_dev(x, torch::kBFloat16, "x");
  check_dev(q, torch::kInt32, "weight");
  check_dev(sz, torch::kInt32, "scales_and_zeros");
  TORCH_CHECK(q.dim() == 2 && sz.dim() == 2 && sz.size(0) == q.size(0) && sz.size(1) * 16 == q.size(1),
              "weight [N, K / 8], scales_and_zeros [N, K / 128]");
  const int64_t n = q.size(0), k = q.size(1) * 8;
  TORCH_CHECK(x.size(-1) == k, "x: last dimension ", k);
  const int64_t m = x.numel() / k;
  auto sizes = x.sizes().vec();
  sizes.back() = n;
  auto y = torch::empty(sizes, x.options());
  auto* xp = reinterpret_cast<const uint16_t*>(x.data_ptr());
  auto* yp = reinterpret_cast<uint16_t*>(y.data_ptr());
  auto* qp = reinterpret_cast<const uint32_t*>(q.data_ptr());
  auto* sp = reinterpret_cast<const uint32_t*>(sz.data_ptr());
  const int rc = m == 1 ? fl_gemv_int4(qp, sp, xp, yp, (int32_t)n, (int32_t)k, stream_of(stream))
                        : fl_gemm_int4(qp, sp, xp, yp, (int32_t)m, (int32_t)n, (int32_t)k, stream_of(stream));
  check_rc(rc, m == 1 ? "fl_gemv_int4" : "fl_gemm_int4");
  return y;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "flint_amd torch ops: the C ABI of libflint_amd.so over torch tensors";
  pybind11::class_<Engine>(m, "Engine")
      .def(pybind11::init<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                          torch::Tensor, torch::Tensor, torch::Tensor, double, double, double, double, double>())
      .def("decode_hidden", &Engine::decode_hidden)
      .def("decode_step", &Engine::decode_step)
      .def("verify", &Engine::verify)
      .def("check", &Engine::check);
  m.def("int4_linear", &int4_linear);
  m.def("version", []() { return fl_version(); });
}
