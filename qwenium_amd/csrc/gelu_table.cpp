// gelu_table.cpp -- the fp16 GeLU table of ggml's CPU backend, on the host and
// once per device.
//
// ggml (llama.cpp tag b8390, vec.h ggml_vec_gelu_f32 with GGML_GELU_FP16, the
// table filled at CPU-backend init) evaluates gelu(x) for -10 < x < 10 as the
// entry at fp16(x) of a 65536-entry table holding fp16(gelu_f32(x16)), where
//     gelu_f32(x) = 0.5*x*(1 + tanh(sqrt(2/pi)*x*(1 + 0.044715*x*x)))
// is evaluated in f32 with the C library's tanhf (the reference's own test,
// tests/unit/test_ffn.cpp:172-175, notes the table).  The same f32 expression
// is evaluated here, so on the same C library the entries are the same bits;
// the GeGLU kernels read the device copy.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "qmoe.h"
#include "qmoe_internal.h"

namespace qmoe {
namespace {

// IEEE binary16 <-> binary32, round to nearest even (all 2^16 codes).
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);  // inf / nan
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        bits = sign;
    } else {  // subnormal: normalize
        int e = -1;
        do {
            ++e;
            mant <<= 1;
        } while (!(mant & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;  // rounds past 65504: inf
    if (ax < 0x38800000u) {                       // below the smallest normal 2^-14
        if (ax < 0x33000000u) return sign;        // below half the smallest subnormal
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;          // 14..24: value = m * 2^(e-150), unit 2^-24
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return sign | (uint16_t)q;
    }
    uint32_t v = ((ax >> 13) - (112u << 10));     // rebias 127 -> 15
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;
    return sign | (uint16_t)v;
}

float gelu_f32(float x) {
#pragma clang fp contract(off)
    const float a = 0.044715f;
    const float c = 0.79788456080286535587989211986876f;  // sqrt(2/pi)
    return 0.5f * x * (1.0f + std::tanh(c * x * (1.0f + a * x * x)));
}

const std::vector<uint16_t>& host_table() {
    static const std::vector<uint16_t> tab = [] {
        std::vector<uint16_t> t(65536);
        for (uint32_t i = 0; i < 65536; ++i) {
            const float f = half_to_float((uint16_t)i);
            t[i] = std::isfinite(f) ? float_to_half(gelu_f32(f)) : (uint16_t)i;
        }
        return t;
    }();
    return tab;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint16_t* g_dev_tab[kMaxDevices] = {};

}  // namespace

void gelu_table_host(uint16_t* out) { std::memcpy(out, host_table().data(), 65536 * sizeof(uint16_t)); }

// The table on the current device, uploaded on first use (held until the
// process ends: 128 KiB per device).
hipError_t gelu_table_device(const uint16_t** out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_dev_tab[dev]) {
        void* p = nullptr;
        if ((err = hipMalloc(&p, 65536 * sizeof(uint16_t))) != hipSuccess) return err;
        if ((err = hipMemcpy(p, host_table().data(), 65536 * sizeof(uint16_t), hipMemcpyHostToDevice)) != hipSuccess) {
            (void)hipFree(p);
            return err;
        }
        g_dev_tab[dev] = (uint16_t*)p;
    }
    *out = g_dev_tab[dev];
    return hipSuccess;
}

}  // namespace qmoe

extern "C" int qmoe_gelu_f16_table(uint16_t* out) {
    if (!out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: out expected room for 65536 fp16 values, got null");
    qmoe::gelu_table_host(out);
    return QMOE_OK;
}
