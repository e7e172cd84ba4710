// Host-side pieces of the C ABI: per-thread error messages, launch checks, the device's CU
// count, and the RoPE inverse-frequency tables (float64 on the host, so the device never
// evaluates pow()).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <unordered_map>

#include "common.h"

namespace pie {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(PIE_HIP_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PIE_HIP_OK;
}

int num_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] > 0) return cached[dev];
  std::lock_guard<std::mutex> lk(mu);
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cached[dev] = n;
  return n;
}

namespace {
struct Inflight {
  hipStream_t stream;
  hipEvent_t done;
};
std::mutex g_inflight_mu;
std::unordered_map<const void*, Inflight> g_inflight;

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
}  // namespace

int inflight_check(const void* key, void* stream, const char* what) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (capturing(st)) return PIE_HIP_OK;
  std::lock_guard<std::mutex> lk(g_inflight_mu);
  auto it = g_inflight.find(key);
  if (it == g_inflight.end() || it->second.stream == st) return PIE_HIP_OK;
  if (hipEventQuery(it->second.done) == hipErrorNotReady)
    return set_error(PIE_HIP_EBUSY,
                     "%s: a launch on another stream still uses the same device state (the "
                     "static scratch or the prefill plan); synchronise first, or give each stream "
                     "its own",
                     what);
  return PIE_HIP_OK;
}

void inflight_mark(const void* key, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (capturing(st)) return;
  std::lock_guard<std::mutex> lk(g_inflight_mu);
  auto it = g_inflight.find(key);
  if (it == g_inflight.end()) {
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return;
    it = g_inflight.emplace(key, Inflight{st, ev}).first;
  }
  it->second.stream = st;
  (void)hipEventRecord(it->second.done, st);
}

}  // namespace pie

using namespace pie;

extern "C" const char* pie_hip_last_error(void) { return g_err; }

extern "C" int pie_hip_abi_version(void) { return 3; }

// Standard RoPE frequencies, f_i = 1 / (rope_scale * theta^(2i/rd)) (flashinfer's
// apply_rope_pos_ids with rope_scale; metal_rope.metal:63-64 with rope_factor = 1).
extern "C" int pie_hip_rope_inv_freq(float* inv_freq, int64_t rotary_dim, float rope_scale,
                                     float rope_theta) {
  PIE_REQUIRE(inv_freq && rotary_dim > 0 && rotary_dim % 2 == 0, "rope_inv_freq: bad rotary_dim");
  PIE_REQUIRE(rope_theta > 0.f && rope_scale > 0.f, "rope_inv_freq: theta and scale must be positive");
  for (int64_t i = 0; i < rotary_dim / 2; ++i)
    inv_freq[i] = (float)(1.0 / ((double)rope_scale * pow((double)rope_theta, (2.0 * i) / (double)rotary_dim)));
  return PIE_HIP_OK;
}

// Llama-3.1 wavelength-based scaling (metal_rope.metal:63-89, flashinfer_metal/ops.py:306-346).
extern "C" int pie_hip_llama31_inv_freq(float* inv_freq, int64_t rotary_dim, float rope_scale,
                                        float rope_theta, float low_freq_factor,
                                        float high_freq_factor, float old_context_len) {
  PIE_REQUIRE(inv_freq && rotary_dim > 0 && rotary_dim % 2 == 0, "llama31_inv_freq: bad rotary_dim");
  PIE_REQUIRE(rope_theta > 0.f && rope_scale > 0.f && old_context_len > 0.f,
              "llama31_inv_freq: theta, scale and old_context_len must be positive");
  PIE_REQUIRE(high_freq_factor > low_freq_factor && low_freq_factor > 0.f,
              "llama31_inv_freq: need 0 < low_freq_factor < high_freq_factor");
  const double L = old_context_len, lo = low_freq_factor, hi = high_freq_factor, s = rope_scale;
  const double low_wavelen = L / lo, high_wavelen = L / hi;
  for (int64_t i = 0; i < rotary_dim / 2; ++i) {
    const double f = 1.0 / pow((double)rope_theta, (2.0 * i) / (double)rotary_dim);
    const double wavelen = 2.0 * M_PI / f;
    double g;
    if (wavelen > low_wavelen) g = f / s;
    else if (wavelen < high_wavelen) g = f;
    else {
      const double smooth = (L / wavelen - lo) / (hi - lo);
      g = (1.0 - smooth) * f / s + smooth * f;
    }
    inv_freq[i] = (float)g;
  }
  return PIE_HIP_OK;
}
