// ABI utilities: thread-local error text, launch checks, ABI version and the device peak table.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <cmath>
#include <mutex>

#include "dtattn_common.hpp"

namespace dtattn {

static thread_local char g_last_error[512] = "";

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DTATTN_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
    return DTATTN_OK;
}

// torch::scaled_dot_product_attention takes any scale (scaled_dot_product_attention_op.cc:107-109 forwards
// SdpaParam's std::optional<double>): logits = scale * q.k (+ mask).  With q negated the logits of
// |scale| are those of a negative scale; with q zeroed every logit is 0 (+ mask), as at scale 0.
int plan_scale(float scale, int64_t D, uint32_t sign_bits, ScalePlan* out) {
    if (std::isnan(scale)) {
        // 1/sqrt(D) in double, rounded once to float: libtorch's default scale, and the value a caller gets
        // by passing 1/sqrt(D) explicitly (an fp32 quotient of an fp32 root differs in the last bit for some
        // D, e.g. 96 and 300)
        *out = ScalePlan{(float)(1.0 / std::sqrt((double)D)), 0xffffffffu, 0u};
        return DTATTN_OK;
    }
    if (std::isinf(scale)) return fail(DTATTN_ERR_INVALID_ARGUMENT, "scale must be finite (NaN selects 1/sqrt(D))");
    if (scale > 0.f) *out = ScalePlan{scale, 0xffffffffu, 0u};
    else if (scale < 0.f) *out = ScalePlan{-scale, 0xffffffffu, sign_bits};
    else *out = ScalePlan{1.0f, 0u, 0u};
    return DTATTN_OK;
}

// Per-device property cache, filled once per device under std::call_once.
namespace {
constexpr int kMaxDevices = 64;
struct PeakCache {
    std::once_flag once[kMaxDevices];
    dtattn_device_peaks peaks[kMaxDevices];
    int status[kMaxDevices];
};
PeakCache& peak_cache() {
    static PeakCache c;
    return c;
}
}  // namespace

}  // namespace dtattn

using namespace dtattn;

extern "C" const char* dtattn_last_error(void) { return g_last_error; }

extern "C" int dtattn_abi_version(void) { return DTATTN_ABI_VERSION; }

extern "C" int dtattn_get_device_peaks(int32_t device, dtattn_device_peaks* out) {
    if (out == nullptr) return fail(DTATTN_ERR_INVALID_ARGUMENT, "peaks: out is NULL");
    if (device < 0 || device >= kMaxDevices) return fail(DTATTN_ERR_INVALID_ARGUMENT, "peaks: bad device %d", device);
    PeakCache& c = peak_cache();
    std::call_once(c.once[device], [&]() {
        hipDeviceProp_t prop;
        hipError_t e = hipGetDeviceProperties(&prop, device);
        if (e != hipSuccess) {
            c.status[device] = DTATTN_ERR_DEVICE;
            return;
        }
        int clock_khz = 0;
        if (hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeClockRate, device) != hipSuccess) clock_khz = 0;
        dtattn_device_peaks pk;
        memset(&pk, 0, sizeof(pk));
        pk.cu_count = prop.multiProcessorCount;
        pk.clock_hz = clock_khz * 1e3;
        // CDNA4 dense MFMA rates per CU per clock: bf16/fp16 4096 FLOP, fp8 8192 FLOP.
        pk.bf16_flops = (double)pk.cu_count * pk.clock_hz * 4096.0;
        pk.fp8_flops = (double)pk.cu_count * pk.clock_hz * 8192.0;
        pk.hbm_bytes_per_s = 8.0e12;  // MI355X HBM3E
        snprintf(pk.arch, sizeof(pk.arch), "%s", prop.gcnArchName);
        c.peaks[device] = pk;
        c.status[device] = DTATTN_OK;
    });
    if (c.status[device] != DTATTN_OK) return fail(DTATTN_ERR_DEVICE, "peaks: hipGetDeviceProperties failed");
    *out = c.peaks[device];
    return DTATTN_OK;
}
