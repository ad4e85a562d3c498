// nnhip_linear_w8a32_noalloc: nnhip_linear_w8a32 for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).  Its scratch -- the weight codes in the
// MFMA operand layout, the activation digit planes and row exponents -- lives
// in one fixed device array, `scratch`, of kNoAllocScratchBytes, which every
// GPU the library runs on holds until the process ends.  Each device's copy
// has its own address, resolved once per device by noalloc_setup (called by
// nnhip_init with that device current); host code uses only that address.
// One context at a time owns a device's array: calls from another context
// on the same GPU (another stream, which nothing would order against the
// owner's) are refused until the owner is destroyed.
#include "api_common.hpp"

#include <mutex>

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;  // 32 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) int8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_dev[kMaxDevices] = {};
const nnhip_ctx *g_scratch_owner[kMaxDevices] = {};

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

namespace nnhip {

void noalloc_setup(int device) {
  NNHIP_REQUIRE(device >= 0 && device < kMaxDevices, kErrArg,
                "noalloc scratch: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[device]) return;
  void *p = nullptr;
  NNHIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  NNHIP_REQUIRE(p != nullptr, kErrHip, "noalloc scratch: no device address");
  g_scratch_dev[device] = p;
}

void noalloc_release(const nnhip_ctx *ctx) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  for (auto &o : g_scratch_owner)
    if (o == ctx) o = nullptr;
}

}  // namespace nnhip

using nnhip::guard;

extern "C" {

int nnhip_linear_w8a32_noalloc(nnhip_ctx *ctx, const float *x, int rows,
                               int K, const int8_t *codes, const float *scales,
                               const float *bias, int N, float *y, int path) {
  return guard([&] {
    NNHIP_REQUIRE(ctx && x && codes && scales && bias && y && rows > 0 && K > 0 &&
                      N > 0,
                  nnhip::kErrArg, "nnhip_linear_w8a32_noalloc: bad argument");
    NNHIP_REQUIRE(path >= 0 && path <= 4, nnhip::kErrArg, "unknown path");
    NNHIP_CHECK(hipSetDevice(ctx->c.device));
    void *base = nullptr;
    bool mine = false;
    {
      std::lock_guard<std::mutex> lk(g_scratch_mu);
      base = g_scratch_dev[ctx->c.device];
      const nnhip_ctx *&owner = g_scratch_owner[ctx->c.device];
      if (!owner) owner = ctx;
      mine = owner == ctx;
    }
    NNHIP_REQUIRE(base, nnhip::kErrHip,
                  "nnhip_linear_w8a32_noalloc: scratch not set up for this device");
    NNHIP_REQUIRE(mine, nnhip::kErrArg,
                  "nnhip_linear_w8a32_noalloc: this GPU's scratch belongs to "
                  "another context (calls on two streams would race on it)");
    hipStream_t st = ctx->c.stream;
    const bool mfma_ok = K % 128 == 0 && N % 64 == 0;
    const bool lds = path == 3 || path == 4;
    const bool mfma = path == 2 || (path == 0 && rows >= 16 && mfma_ok);
    NNHIP_REQUIRE(!(path == 2 && !mfma_ok), nnhip::kErrArg,
                  "MFMA path needs K % 128 == 0 and N % 64 == 0");
    NNHIP_REQUIRE(!lds || nnhip::gemm_lds_supports(rows, K, N), nnhip::kErrArg,
                  "LDS GEMM needs K in {128, 256, 512, 1024} and N % 32 == 0");
    if (!lds && !mfma) {
      // the GEMV reads the caller's codes directly: no scratch
      nnhip::launch_gemv(st, x, K, rows, K, N, codes, nullptr, scales, bias,
                         nullptr, 0, y, N, nnhip::kEpiBias);
      return;
    }
    // scratch: [swizzled codes N*K][digits 3*mpad*K][row exponents mpad]
    const int mpad = (rows + 63) / 64 * 64;
    const size_t sw_bytes = align256((size_t)N * K);
    const size_t limb_bytes = align256((size_t)3 * mpad * K);
    const size_t need = sw_bytes + limb_bytes + (size_t)mpad * sizeof(int);
    NNHIP_REQUIRE(need <= kNoAllocScratchBytes, nnhip::kErrArg,
                  "nnhip_linear_w8a32_noalloc: N*K + 3*K*rows64 + 4*rows64 "
                  "bytes of scratch exceed its fixed 32 MiB");
    int8_t *sw = static_cast<int8_t *>(base);
    int8_t *limbs = sw + sw_bytes;
    int *rexp = reinterpret_cast<int *>(limbs + limb_bytes);
    nnhip::launch_swizzle_rows(st, codes, N, K, sw, false);
    if (lds) {
      if (path == 4) nnhip::launch_act_quant(st, x, K, rows, K, limbs, mpad, rexp);
      nnhip::launch_gemm_lds(st, path == 4 ? nnhip::kAFromDigits : nnhip::kAFromRows,
                             limbs, mpad, rexp, x, K, nullptr, nullptr, nullptr,
                             0, rows, K, N, sw, scales, bias, nullptr, 0, y, N,
                             nnhip::kEpiBias);
    } else {
      nnhip::launch_act_quant(st, x, K, rows, K, limbs, mpad, rexp);
      nnhip::launch_gemm_limb(st, limbs, mpad, rexp, rows, K, N, sw, scales,
                              bias, nullptr, 0, y, N, nnhip::kEpiBias);
    }
  });
}

}  // extern "C"
