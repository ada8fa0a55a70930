// xitem.h -- 8 activation elements of one source dtype (fp16 / bf16 / fp32),
// loaded with 16-byte loads and converted to fp16 for an LDS stage.
#pragma once

#include "common.h"

namespace tq {

typedef _Float16 xh2_t __attribute__((ext_vector_type(2)));

// 8 activation elements of one source dtype, converted to fp16 for LDS.
template <int XDT>
struct XItem;
template <>
struct XItem<TITAN_FP16> {
    uint4 a;
    TQ_DEV void load(const void* p, int64_t e) { a = *(const uint4*)((const uint16_t*)p + e); }
    TQ_DEV void zero() { a = make_uint4(0, 0, 0, 0); }
    TQ_DEV uint4 h() const { return a; }
};
template <>
struct XItem<TITAN_BF16> {
    uint4 a;
    TQ_DEV void load(const void* p, int64_t e) { a = *(const uint4*)((const uint16_t*)p + e); }
    TQ_DEV void zero() { a = make_uint4(0, 0, 0, 0); }
    TQ_DEV static uint32_t cv(uint32_t w) {
        const xh2_t v = {(_Float16)bf16_to_f32(w & 0xFFFFu), (_Float16)bf16_to_f32(w >> 16)};
        return __builtin_bit_cast(uint32_t, v);
    }
    TQ_DEV uint4 h() const { return make_uint4(cv(a.x), cv(a.y), cv(a.z), cv(a.w)); }
};
template <>
struct XItem<TITAN_FP32> {
    float4 a, b;
    TQ_DEV void load(const void* p, int64_t e) {
        a = *(const float4*)((const float*)p + e);
        b = *(const float4*)((const float*)p + e + 4);
    }
    TQ_DEV void zero() { a = b = make_float4(0, 0, 0, 0); }
    TQ_DEV static uint32_t cv(float x, float y) {
        const xh2_t v = {(_Float16)x, (_Float16)y};
        return __builtin_bit_cast(uint32_t, v);
    }
    TQ_DEV uint4 h() const { return make_uint4(cv(a.x, a.y), cv(a.z, a.w), cv(b.x, b.y), cv(b.z, b.w)); }
};

}  // namespace tq
