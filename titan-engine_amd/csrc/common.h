// common.h -- shared device/host helpers for the gfx950 quantized matmul path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "titan_qmm.h"

#define TQ_DEV __device__ __forceinline__
#define TQ_HD __host__ __device__ __forceinline__

namespace tq {

// 16-byte load of data that a kernel streams once (quantized weight codes):
// nontemporal, measured faster than cached loads for the GEMV, the
// token-tiled GEMM and the MoE expert GEMM (TQ_STREAM_CACHED restores plain
// loads, for comparison)
#ifndef TQ_STREAM_CACHED
typedef uint32_t tq_u32x4 __attribute__((ext_vector_type(4)));
TQ_DEV uint4 ld_stream_u128(const void* p) {
    const tq_u32x4 v = __builtin_nontemporal_load((const tq_u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
#else
TQ_DEV uint4 ld_stream_u128(const void* p) { return *(const uint4*)p; }
#endif
template <bool NT>
TQ_DEV uint4 ld_codes_u128(const void* p) {
    if constexpr (NT) return ld_stream_u128(p);
    else return *(const uint4*)p;
}

constexpr int kWave = 64;

// ---- scalar conversions (bit-exact, no library math) -----------------------

TQ_DEV float f16_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;  // v_cvt_f32_f16: exact, subnormals included
}
TQ_DEV float bf16_to_f32(uint32_t h) { return __builtin_bit_cast(float, h << 16); }
TQ_DEV uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
TQ_DEV uint16_t f32_to_f16_rne(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32 rounds to nearest even
}

// E4M3 (bias 7) as the reference decodes scales: fp4.cu:173-185, the two NaN
// codes (0x7F, 0xFF) read as 0.  Built from bits: no ldexp.
TQ_DEV float e4m3_ref_to_f32(uint32_t v) {
    v &= 0xFF;
    uint32_t mag = v & 0x7F;
    uint32_t e = mag >> 3, m = mag & 7;
    // normal: 2^(e-7) * (1 + m/8) -> fp32 exponent e + 120, mantissa m << 20
    // subnormal (e == 0): m * 2^-9 (exact integer scaling)
    float f = e ? __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20))
                : (float)m * 0.001953125f;
    f = (mag == 0x7F) ? 0.0f : f;
    return (v & 0x80) ? -f : f;
}

// E2M1 magnitude table of fp4.cu:23-26 built from bits: code c (sign in bit 3)
// -> fp32.  e = (c>>1)&3, m = c&1: e ? (1 + m/2) 2^(e-1) : m/2.
TQ_DEV float fp4_to_f32(uint32_t c) {
    uint32_t e = (c >> 1) & 3u, m = c & 1u;
    uint32_t bits = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
    return __builtin_bit_cast(float, bits | ((c & 8u) << 28));
}

// OCP E4M3FN (gfx950 fp8) -> fp32 for weights; same values as the reference
// decoder except the NaN codes.
TQ_DEV float e4m3_ocp_to_f32(uint32_t v) {
    v &= 0xFF;
    if ((v & 0x7F) == 0x7F) return __builtin_nanf("");
    return e4m3_ref_to_f32(v);
}

// Round-to-nearest-even, saturating fp32 -> e4m3 (finite inputs); the same
// algorithm as the CPU oracle so that activation codes match bit for bit.
TQ_DEV uint32_t f32_to_e4m3_rne_sat(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (u >> 24) & 0x80u;
    float a = __builtin_fabsf(f);
    if (a != a) return 0x7Fu;
    if (a >= 448.0f) return sign | 0x7Eu;
    if (a < 0.015625f) {
        float m = __builtin_rintf(a * 512.0f);
        return sign | (uint32_t)m;
    }
    uint32_t au = __builtin_bit_cast(uint32_t, a);
    int E = (int)(au >> 23) - 127;  // a in [2^E, 2^(E+1)), E in [-6, 8]
    float t = (__builtin_bit_cast(float, (au & 0x807FFFFFu) | 0x3F800000u) - 1.0f) * 8.0f;
    int mi = (int)__builtin_rintf(t);
    if (mi == 8) { mi = 0; E += 1; }
    if (E > 8 || (E == 8 && mi > 6)) return sign | 0x7Eu;
    return sign | (uint32_t)(((E + 7) << 3) | mi);
}

// ---- activation load / output store by runtime dtype -------------------------

TQ_DEV float load_act(const void* p, int64_t i, int dt) {
    if (dt == TITAN_FP32) return ((const float*)p)[i];
    uint32_t h = ((const uint16_t*)p)[i];
    return dt == TITAN_FP16 ? f16_to_f32(h) : bf16_to_f32(h);
}
TQ_DEV void store_out(void* p, int64_t i, int dt, float v) {
    if (dt == TITAN_FP32) ((float*)p)[i] = v;
    else if (dt == TITAN_FP16) ((uint16_t*)p)[i] = f32_to_f16_rne(v);
    else ((uint16_t*)p)[i] = f32_to_bf16_rne(v);
}

// ---- wave reductions -------------------------------------------------------
// Sum over the four lanes {l, l^16, l^32, l^48} (the four slots of a row).
TQ_DEV float sum_slots(float v) {
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}
TQ_DEV float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

}  // namespace tq

// ---- host-side validation helpers ----------------------------------------------
namespace tqh {
inline bool act_dtype_ok(int dt) {
    return dt == TITAN_FP32 || dt == TITAN_FP16 || dt == TITAN_BF16;
}
inline int launch_status() {
    return hipGetLastError() == hipSuccess ? TITAN_OK : TITAN_ERR_LAUNCH;
}
}  // namespace tqh
