// Drop-in device counterparts of the reference's decoder objects, over
// libnnhip.so's C ABI (include/nnhip.h).  Compiled against the reference's
// headers; a program using them links the reference's own nn / core
// sources, as any other user of TransformerDecoder does.
//
//   reference                                   here
//   TransformerDecoder (layer.hpp:299-330)       HipDecoder (mirrors one by
//                                                its parameters())
//   TransformerDecoder::forward(x, caches)       HipDecoder::forward(ids,
//     (layer.cpp:1161-1193)                      HipKVCache *)
//   KVCache / KVCache::truncate (layer.hpp:      HipKVCache / truncate
//     212-230, layer.cpp:67-149)
//   quantize_model (quantization.hpp:43) over    HipDecoder::quantize
//     every Dense of the decoder
//   QuantizedDense::forward (quantization.cpp:   HipQuantizedDense::forward
//     127-147)
//   MultiHeadAttention::forward(x, KVCache *)    HipMultiHeadAttention::forward
//     (layer.cpp:593-994)                        (x, HipMhaCache *)
//   generate_advanced (layer.hpp:310-316)        HipDecoder::generate_advanced
//   generate_speculative (layer.hpp:318-323)     HipDecoder::generate_speculative
//
// Sampled generation draws from std::mt19937 seeded with the seed, in the
// reference's order and with libstdc++'s draws (HipBackend sets the
// library's "rng" option to 1 on its context).
#pragma once

#include "hip_backend.hpp"
#include "nn/layer.hpp"
#include "nn/quantization.hpp"

#include <memory>
#include <vector>

namespace nnhip_backend {

// TransformerDecoder's constructor arguments (layer.hpp:300-302), which the
// decoder does not expose
struct DecoderConfig {
  size_t vocab_size, embed_dim, num_heads, dim_feedforward, num_layers,
      max_seq_len;
};

class HipKVCache;

class HipDecoder {
 public:
  // copies d.parameters() (layer.cpp:1140-1154, same order) to the device
  HipDecoder(HipBackend &backend, TransformerDecoder &d,
             const DecoderConfig &cfg);
  // the same from host arrays in parameters() order (the shapes of
  // nnhip_decoder_param_shape), for programs that hold the weights without
  // a TransformerDecoder object (e.g. read from a file)
  HipDecoder(HipBackend &backend, const DecoderConfig &cfg,
             const std::vector<std::vector<float>> &params);
  ~HipDecoder();
  HipDecoder(const HipDecoder &) = delete;
  HipDecoder &operator=(const HipDecoder &) = delete;

  // every Dense (q, k, v, o, gate, up, down, lm_head) to symmetric codes per
  // output channel with the QuantizedDense formula (quantization.cpp:36-86):
  // config.type INT8 (max|w| / 127) or INT4 (max|w| / 7), as quantize_model
  // takes it (quantization.hpp:8-12, 43)
  void quantize(const QuantizationConfig &config = QuantizationConfig{});
  // logits [S][V] of one sequence of ids [S]; cache may be null
  std::vector<float> forward(const std::vector<size_t> &ids,
                             HipKVCache *cache);
  std::vector<size_t> generate_advanced(const std::vector<size_t> &prompt,
                                        size_t max_new_tokens,
                                        float temperature = 1.0f,
                                        size_t top_k = 0, float top_p = 1.0f,
                                        unsigned int seed = 42,
                                        bool use_kv_cache = true);
  std::vector<size_t>
  generate_speculative(HipDecoder *draft_model,
                       const std::vector<size_t> &prompt, size_t max_new_tokens,
                       size_t lookahead = 4, float temperature = 1.0f,
                       size_t top_k = 0, float top_p = 1.0f,
                       unsigned int seed = 42, bool quantized_cache = false);
  [[nodiscard]] nnhip_model *handle() const noexcept { return m_; }
  [[nodiscard]] const DecoderConfig &config() const noexcept { return cfg_; }

 private:
  nnhip_model *m_ = nullptr;
  DecoderConfig cfg_;
};

// KVCache(quantized) for one sequence of a HipDecoder
class HipKVCache {
 public:
  HipKVCache(HipDecoder &model, bool quantized = false);
  ~HipKVCache();
  HipKVCache(const HipKVCache &) = delete;
  HipKVCache &operator=(const HipKVCache &) = delete;
  void truncate(size_t len);
  [[nodiscard]] size_t length() const;
  [[nodiscard]] nnhip_kvcache *handle() const noexcept { return c_; }

 private:
  nnhip_kvcache *c_ = nullptr;
};

// MultiHeadAttention's constructor arguments (layer.hpp:234-236)
struct MhaConfig {
  size_t embed_dim, num_heads;
  size_t num_kv_heads = 0;   // 0: num_heads (layer.cpp:475)
  bool causal = true;        // the device attention is causal (the decoder's)
  size_t max_seq_len = 1024; // capacity of a HipMhaCache
};

class HipMhaCache;

// MultiHeadAttention (layer.hpp:232-258, layer.cpp:471-994) on the device:
// q / k / v projections as one fused Linear (fp32, or INT8 / INT4 codes
// after quantize), RoPE at the cache's length and the KV append
// (nnhip_rope_kv_append_gqa), the fused causal attention with grouped
// query heads (nnhip_attention_kq), the output projection.
class HipMultiHeadAttention {
 public:
  // parameters in MultiHeadAttention::parameters() order (layer.cpp:491-502):
  // q, k, v, out projections, each weight [in][out] then bias [out]
  HipMultiHeadAttention(HipBackend &backend, const MhaConfig &cfg,
                        const std::vector<std::vector<float>> &params);
  // the same from a reference layer (its parameters() copied to the host)
  HipMultiHeadAttention(HipBackend &backend, MultiHeadAttention &layer,
                        const MhaConfig &cfg);
  ~HipMultiHeadAttention();
  HipMultiHeadAttention(const HipMultiHeadAttention &) = delete;
  HipMultiHeadAttention &operator=(const HipMultiHeadAttention &) = delete;

  // MultiHeadAttention::quantize (layer.cpp:545-558): every projection to
  // symmetric per-output-channel codes, INT8 or INT4
  void quantize(const QuantizationConfig &config = QuantizationConfig{});
  // forward(x, cache) on device rows: x [B*S][E] -> y [B*S][E] (E =
  // embed_dim), B sequences of S new positions; cache may be null (no
  // past), else holds B sequences and grows by S
  void forward_device(const float *x, size_t B, size_t S, float *y,
                      HipMhaCache *cache);
  // forward(input [B, S, E], cache) on HipBackend tensors
  std::shared_ptr<Tensor> forward(const std::shared_ptr<Tensor> &input,
                                  HipMhaCache *cache = nullptr);
  [[nodiscard]] const MhaConfig &config() const noexcept { return cfg_; }
  [[nodiscard]] size_t head_dim() const noexcept { return D_; }
  [[nodiscard]] size_t kv_heads() const noexcept { return Hkv_; }

 private:
  friend class HipMhaCache;
  HipBackend &be_;
  MhaConfig cfg_;
  size_t H_ = 0, Hkv_ = 0, D_ = 0;
  bool quantized_ = false;
  // fused q | k | v: fp32 [Nqkv][E] or codes, scales, bias [Nqkv]; out: [E][E]
  std::unique_ptr<DeviceBuffer> wqkv_, wo_, cqkv_, co_, sqkv_, so_, bqkv_, bo_;
  std::vector<std::vector<float>> master_;  // parameters() as given
  // forward scratch (q | k | v rows, rotated q, context rows, positions),
  // kept across calls for up to s_rows_ rows of s_B_ sequences
  std::unique_ptr<DeviceBuffer> s_qkv_, s_qrot_, s_ctx_, s_pos_;
  size_t s_rows_ = 0, s_B_ = 0;
};

// KVCache for B sequences of one HipMultiHeadAttention: fp32 K / V
// [B][Hkv][max_seq_len][D] on the device, one length for all sequences as
// the reference's cache has (layer.hpp:212-230).
class HipMhaCache {
 public:
  HipMhaCache(HipMultiHeadAttention &layer, size_t batch);
  void truncate(size_t len);  // KVCache::truncate (layer.cpp:67-149)
  [[nodiscard]] size_t length() const noexcept { return len_; }
  [[nodiscard]] size_t batch() const noexcept { return B_; }

 private:
  friend class HipMultiHeadAttention;
  size_t B_ = 0, cap_ = 0, len_ = 0;
  std::unique_ptr<DeviceBuffer> k_, v_;
};

// QuantizedDense (INT8 or INT4, quantization.hpp:15-41, quantization.cpp:
// 7-147) on device pointers: the codes, scales and bias resident on the
// device, the reference's packed_weights layout on the host.  Uses no
// compiled reference code (hip_qdense.cpp), so programs run it without the
// reference's sources; HipQuantizedDense is the same over Tensor.
class HipQuantizedDenseCore {
 public:
  // QuantizedDense(float_dense, config) (quantization.cpp:7-86): weight
  // [in][out] (Dense's layout) and bias [out] on the host, quantised on the
  // device (nnhip_quantize_w8 / _w4): the reference's codes and scales bit
  // for bit
  HipQuantizedDenseCore(HipBackend &backend, const std::vector<float> &weight,
                        size_t in, size_t out, const std::vector<float> &bias,
                        QuantizationType type);
  // the packed_weights, scales and bias of a reference QuantizedDense
  HipQuantizedDenseCore(HipBackend &backend, QuantizationType type, size_t in,
                        size_t out, const std::vector<uint8_t> &packed,
                        const std::vector<float> &scales,
                        const std::vector<float> &bias);
  // forward (quantization.cpp:127-147) on device rows: y [rows][out] =
  // x [rows][in] . (codes * scales) + bias, enqueued on the backend's stream
  void forward_device(const float *x, size_t rows, float *y) const;
  // dequantize_weight (quantization.cpp:89-125): codes * scales, [in][out]
  [[nodiscard]] std::vector<float> dequantize_weight() const;
  [[nodiscard]] QuantizationType type() const noexcept { return type_; }
  [[nodiscard]] const std::vector<uint8_t> &packed_weights() const noexcept {
    return packed_;
  }
  [[nodiscard]] const std::vector<float> &scales() const noexcept {
    return host_scales_;
  }
  [[nodiscard]] const std::vector<float> &bias() const noexcept {
    return host_bias_;
  }
  [[nodiscard]] size_t in_features() const noexcept { return in_; }
  [[nodiscard]] size_t out_features() const noexcept { return out_; }
  [[nodiscard]] HipBackend &backend() const noexcept { return be_; }

 private:
  void upload(const std::vector<int8_t> &codes_in_out,
              const std::vector<float> &scales, const std::vector<float> &bias);
  HipBackend &be_;
  QuantizationType type_ = QuantizationType::INT8;
  size_t in_ = 0, out_ = 0;
  std::vector<uint8_t> packed_;                           // reference layout
  std::vector<int8_t> host_codes_;                        // [in][out]
  std::vector<float> host_scales_, host_bias_;
  std::unique_ptr<DeviceBuffer> codes_, scales_, bias_;  // codes [out][in]
};

// HipQuantizedDenseCore over Tensor: forward runs on tensors whose storage
// belongs to `backend` (hip_nn.cpp, linked with the reference's sources).
class HipQuantizedDense {
 public:
  // the codes and scales of a reference QuantizedDense
  HipQuantizedDense(HipBackend &backend, const QuantizedDense &layer);
  // QuantizedDense(float_dense, config), quantised on the device
  HipQuantizedDense(HipBackend &backend, std::shared_ptr<Dense> float_dense,
                    const QuantizationConfig &config);
  // y [rows, out] = x [rows, in] . (codes * scales) + bias, x contiguous
  std::shared_ptr<Tensor> forward(const std::shared_ptr<Tensor> &input);
  // the accessors of QuantizedDense (quantization.hpp:20-31)
  [[nodiscard]] QuantizationType type() const noexcept { return core_->type(); }
  [[nodiscard]] const std::vector<uint8_t> &packed_weights() const noexcept {
    return core_->packed_weights();
  }
  [[nodiscard]] Shape weight_shape() const {
    return Shape{core_->in_features(), core_->out_features()};
  }
  std::shared_ptr<Tensor> scales() const;  // [out] on the HipBackend
  std::shared_ptr<Tensor> bias() const;    // [1, out] on the HipBackend
  // dequantize_weight (quantization.cpp:89-125): codes * scales, [in, out]
  std::shared_ptr<Tensor> dequantize_weight() const;
  [[nodiscard]] const HipQuantizedDenseCore &core() const noexcept { return *core_; }

 private:
  std::unique_ptr<HipQuantizedDenseCore> core_;
};

}  // namespace nnhip_backend
