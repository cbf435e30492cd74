// Shared device/host helpers for the MI355X (gfx950) paged-attention kernels.
//
// Everything here is written for CDNA4: 64-lane wavefronts, MFMA matrix
// cores (v_mfma_f32_16x16x32_{bf16,f16}, v_mfma_f32_16x16x16{bf16_1k,f16}),
// and 128-bit global loads.  No other target is supported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mstar_amd.h"

#define MI_DEVICE __device__ __forceinline__

namespace mi {

constexpr int kWave = 64;

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef i16x4 v4i16;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// ---------------------------------------------------------------- bit casts
template <typename To, typename From>
MI_DEVICE To bitcast(const From& v) {
  static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
  return __builtin_bit_cast(To, v);
}

// ------------------------------------------------------- scalar conversions
// float -> bfloat16 bits, round-to-nearest-even; NaN -> 0x7FC0 (canonical
// quiet NaN with the input's sign dropped), the same result torch's
// Tensor.to(torch.bfloat16) produces on the CPU.
MI_DEVICE uint16_t f32_to_bf16_rne(float x) {
  uint32_t u = bitcast<uint32_t>(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

MI_DEVICE float bf16_to_f32(uint16_t h) { return bitcast<float>((uint32_t)h << 16); }

// float -> fp16 bits, round-to-nearest-even (hardware v_cvt_f16_f32 uses the
// default RNE mode; overflow -> inf, NaN -> NaN).
MI_DEVICE uint16_t f32_to_f16_rne(float x) { return bitcast<uint16_t>((_Float16)x); }
MI_DEVICE float f16_to_f32(uint16_t h) { return (float)bitcast<_Float16>(h); }

// float -> OCP fp8 e4m3fn (bias 7, no infinities, 0x7F/0xFF = NaN, max 448).
// Round-to-nearest-even.  Magnitudes that round past 448 (>= 464) and NaN
// map to NaN, matching torch's non-saturating float8_e4m3fn cast; callers
// clamp to +-448 first.  Branch-free: both the normal and the subnormal
// result are formed and one is selected.  Normal range: adding 0x7ffff plus
// the lowest kept mantissa bit rounds the 20 dropped bits to nearest-even on
// the bit pattern, a carry moving into the exponent; (bits >> 20) is then
// exponent:mantissa, and subtracting 120 << 3 rebiases 127 -> 7.
MI_DEVICE uint8_t f32_to_e4m3fn(float x) {
  const uint32_t u = bitcast<uint32_t>(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  const uint32_t nrm = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
  // < 2^-6: subnormal grid 2^-9, exact scale then RNE; q == 8 encodes 2^-6.
  const uint32_t sub = (uint32_t)__builtin_rintf(bitcast<float>(a) * 512.0f);
  const uint32_t v = a < 0x3c800000u ? sub : nrm;
  return (uint8_t)(sign | (a >= 0x43e80000u ? 0x7fu : v));  // >= 464.0 or NaN/inf
}

// ------------------------------------------------------------ type traits
// 16-bit floating storage types handled by the MFMA paths.
struct BF16 {
  static constexpr int kDtype = MI_BF16;
  MI_DEVICE static float to_f32(uint16_t h) { return bf16_to_f32(h); }
  MI_DEVICE static uint16_t from_f32(float x) { return f32_to_bf16_rne(x); }
  // Two floats -> packed pair, RNE (hardware v_cvt_pk_bf16_f32 on gfx950).
  MI_DEVICE static uint32_t pack2(float a, float b) {
    const f32x2 v = {a, b};
    return bitcast<uint32_t>(__builtin_convertvector(v, bf16x2));
  }
  // S^T tile product: A = 16x32 (8 elems/lane), B = 32x16, C = 16x16 fp32.
  MI_DEVICE static f32x4 mma_16x16x32(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  }
  // A = 16x16 (4 elems/lane), B = 16x16, C = 16x16 fp32.
  MI_DEVICE static f32x4 mma_16x16x16(const uint2& a, const uint2& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bitcast<i16x4>(a), bitcast<i16x4>(b), c, 0, 0, 0);
  }
  // acc + lo(w) + hi(w) of a packed pair, in one v_dot2.
  MI_DEVICE static float sum2(uint32_t w, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(w), one, acc, false);
  }
};

struct F16 {
  static constexpr int kDtype = MI_F16;
  MI_DEVICE static float to_f32(uint16_t h) { return f16_to_f32(h); }
  MI_DEVICE static uint16_t from_f32(float x) { return f32_to_f16_rne(x); }
  MI_DEVICE static uint32_t pack2(float a, float b) {  // v_cvt_pk_f16_f32, RNE
    const f32x2 v = {a, b};
    return bitcast<uint32_t>(__builtin_convertvector(v, f16x2));
  }
  MI_DEVICE static f32x4 mma_16x16x32(const uint4& a, const uint4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
  MI_DEVICE static f32x4 mma_16x16x16(const uint2& a, const uint2& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(bitcast<f16x4>(a), bitcast<f16x4>(b), c, 0, 0, 0);
  }
  MI_DEVICE static float sum2(uint32_t w, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(bitcast<f16x2>(w), one, acc, false);
  }
};

// fp32 output rows (the merge of fp32 attention writes floats).
struct F32Out {
  static constexpr int kDtype = MI_F32;
};

// fp8 e4m3fn pair (selected 16-bit half of `w`) -> packed 16-bit pair of the
// MFMA type, exact (gfx950 hardware conversion, scale 1.0).
template <typename MT>
MI_DEVICE uint32_t fp8x2_to_mt(uint32_t w, bool hi);
template <>
MI_DEVICE uint32_t fp8x2_to_mt<BF16>(uint32_t w, bool hi) {
  return hi ? bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))
            : bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <>
MI_DEVICE uint32_t fp8x2_to_mt<F16>(uint32_t w, bool hi) {
  return hi ? bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))
            : bitcast<uint32_t>(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}

// ------------------------------------------------------------ lane helpers
MI_DEVICE int lane_id() { return __lane_id(); }

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  In each group of 16
// lanes, lane l receives element l%4 of the 64-bit rows addressed by lanes
// 4k + l/4, k = 0..3 (as element k).  addr must be 8-byte aligned.
MI_DEVICE v4i16 ds_read_tr16(const uint8_t* lds_addr) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds_addr));
}

// Wave-uniform value in an SGPR.
MI_DEVICE int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
MI_DEVICE int64_t uniform64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

MI_DEVICE float xor_shuffle(float v, int mask) { return __shfl_xor(v, mask, kWave); }

// max / sum over the four lanes {l, l^16, l^32, l^48} (the four 16-lane rows
// holding one MFMA column), on the VALU: v_permlane32_swap pairs lane l with
// l^32 and v_permlane16_swap pairs row r with row r^1; taking both outputs of
// each swap makes the result independent of which operand receives which half.
MI_DEVICE float rows4_max(float x) {
  const uint32_t u = bitcast<uint32_t>(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float y = fmaxf(bitcast<float>((uint32_t)a[0]), bitcast<float>((uint32_t)a[1]));
  const uint32_t v = bitcast<uint32_t>(y);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return fmaxf(bitcast<float>((uint32_t)b[0]), bitcast<float>((uint32_t)b[1]));
}
MI_DEVICE float rows4_sum(float x) {
  const uint32_t u = bitcast<uint32_t>(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float y = bitcast<float>((uint32_t)a[0]) + bitcast<float>((uint32_t)a[1]);
  const uint32_t v = bitcast<uint32_t>(y);
  const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return bitcast<float>((uint32_t)b[0]) + bitcast<float>((uint32_t)b[1]);
}

// Streaming (non-temporal) global loads: KV pages are read once per launch.
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
MI_DEVICE uint4 nt_load16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
MI_DEVICE uint2 nt_load8(const void* p) {
  const u32x2_t v = __builtin_nontemporal_load((const u32x2_t*)p);
  return make_uint2(v.x, v.y);
}
MI_DEVICE uint32_t nt_load4(const void* p) { return __builtin_nontemporal_load((const uint32_t*)p); }

// v_perm_b32: byte i of the result = byte sel[i] of {hi:lo} where selector
// values 0-3 address `lo` and 4-7 address `hi`.
MI_DEVICE uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// (lo16(a), lo16(b)) and (hi16(a), hi16(b)) packs.
MI_DEVICE uint32_t pack_lo16(uint32_t a, uint32_t b) { return perm_b32(b, a, 0x05040100u); }
MI_DEVICE uint32_t pack_hi16(uint32_t a, uint32_t b) { return perm_b32(b, a, 0x07060302u); }

MI_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
MI_DEVICE float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace mi

// ------------------------------------------------------------ host helpers
#define MI_CHECK_LAUNCH()                                   \
  do {                                                      \
    hipError_t _e = hipGetLastError();                      \
    if (_e != hipSuccess) return MI_ERR_LAUNCH;             \
  } while (0)

static inline int64_t mi_align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }
