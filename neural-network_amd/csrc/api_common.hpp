// Shared by the C ABI translation units: opaque handle types and the
// exception-to-status guard.
#pragma once

#include "engine.hpp"
#include "nnhip.h"

#include <memory>
#include <string>

struct nnhip_ctx {
  nnhip::Ctx c;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // scratch of the fused entry points, reused in stream order on c.stream:
  // digit planes and row exponents, the codes in the MFMA operand layout
  // (grown when a call needs more, after the stream has drained)
  nnhip::DevBuf<int8_t> limbs, sw;
  nnhip::DevBuf<int> rexp;
  // RoPE cos / sin tables of the standalone append entry points, one per
  // head width, for positions [0, n) (grown, after the stream has drained,
  // when a call needs more positions), and the attention entry point's
  // partial results
  struct Rope {
    int D = 0, n = 0;
    nnhip::DevBuf<float> c, s;
  } rope[4];
  nnhip::DevBuf<float> part;
  // nnhip_spec_accept's state and scratch, kept for the next call of the
  // same (B, k, V) (every call resets the state and synchronizes the stream)
  std::unique_ptr<nnhip::AcceptRows> accept;
  int acc_B = 0, acc_k = 0, acc_V = 0;
};
struct nnhip_model {
  std::unique_ptr<nnhip::Model> m;
};
struct nnhip_kvcache {
  std::unique_ptr<nnhip::KVCache> c;
};

namespace nnhip {

void set_last_error(const std::string &msg);
// resolves this device's copy of the fixed scratch array of
// nnhip_linear_w8a32_noalloc (noalloc.hip); device must be current
void noalloc_setup(int device);
// gives up the scratch array a destroyed context owned
void noalloc_release(const nnhip_ctx *ctx);

template <typename F>
int guard(F &&f) {
  try {
    f();
    return NNHIP_OK;
  } catch (const Error &e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc &) {
    set_last_error("host allocation failed");
    return NNHIP_EHIP;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return NNHIP_EARG;
  }
}

}  // namespace nnhip
