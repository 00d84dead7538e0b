// common.hpp — device helpers shared by the gfx950 kernels: the float32 steps of the reference's kernels done one
// rounding at a time (every file is built with -ffp-contract=off and correctly rounded division and square root),
// the Cephes exponential of kernels/kernel.ts:15-45, the float16 conversions of kernels/kernel.ts:383-392,570-599 and
// the int6 widening of kernels/six.ts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GS 32  // the quantization group (quantize.py)

namespace ple {

// ---- integer helpers ----

// i32.trunc_sat_f32_s: NaN to 0, out of range to the nearest end (the conversion of quantize_x, kernels/kernel.ts:145)
// (as selects: the clamped conversion, then the top end and NaN)
__device__ __forceinline__ int32_t trunc_sat(float f) {
  const float c = __builtin_fminf(__builtin_fmaxf(f, -2147483648.0f), 2147483520.0f);
  int32_t r = (int32_t)c;
  r = f >= 2147483648.0f ? 2147483647 : r;
  return __builtin_isnan(f) ? 0 : r;
}
__device__ __forceinline__ int32_t sat16(int32_t v) { return v > 32767 ? 32767 : (v < -32768 ? -32768 : v); }
__device__ __forceinline__ int32_t sat8(int32_t v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }

// quantize_x's value: narrow(trunc_sat(nearest(x * inv)) + bias) (kernels/kernel.ts:145-153; the i32 add wraps)
__device__ __forceinline__ int8_t quant_value(float x, float inv, int32_t bias) {
  const int32_t t = (int32_t)((uint32_t)trunc_sat(__builtin_rintf(x * inv)) + (uint32_t)bias);
  return (int8_t)sat8(sat16(t));
}

// four activations of quantize_x(bias 64) with the bias taken out, q - 64 per byte: (q + 0x40) ^ 0x80 for q in
// 0..127 (no carry leaves a byte). dot(w, q - 64) is matmul_q8r's group sum with int8_sums' correction in it
// (kernels/kernel_relaxed.ts:47-55, kernels/kernel.ts:204-212).
__device__ __forceinline__ uint32_t centre4(uint32_t q) { return (q + 0x40404040u) ^ 0x80808080u; }

__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// kernels/six.ts: a group's 24 bytes (low nibbles in bytes 0..15, the top two bits of values k, k+8, k+16, k+24 in
// byte 16+k at bits 0, 2, 4, 6) widened to its 32 int8 values (multiples of 4), four a word
__device__ __forceinline__ void six_widen(const uint32_t L[4], uint32_t T0, uint32_t T1, uint32_t w[8]) {
  w[0] = ((L[0] & 0x0F0F0F0Fu) << 2) | ((T0 & 0x03030303u) << 6);
  w[1] = ((L[1] & 0x0F0F0F0Fu) << 2) | ((T1 & 0x03030303u) << 6);
  w[2] = ((L[2] & 0x0F0F0F0Fu) << 2) | ((T0 << 4) & 0xC0C0C0C0u);
  w[3] = ((L[3] & 0x0F0F0F0Fu) << 2) | ((T1 << 4) & 0xC0C0C0C0u);
  w[4] = ((L[0] >> 2) & 0x3C3C3C3Cu) | ((T0 << 2) & 0xC0C0C0C0u);
  w[5] = ((L[1] >> 2) & 0x3C3C3C3Cu) | ((T1 << 2) & 0xC0C0C0C0u);
  w[6] = ((L[2] >> 2) & 0x3C3C3C3Cu) | (T0 & 0xC0C0C0C0u);
  w[7] = ((L[3] >> 2) & 0x3C3C3C3Cu) | (T1 & 0xC0C0C0C0u);
}

// ---- float helpers ----

__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }

// f32x4.max / f32x4.min of WebAssembly: NaN if either is, else the larger / smaller (+0 above -0); written as
// selects, so that no branch splits a wave
__device__ __forceinline__ float wmax(float a, float b) {
  const float larger = a > b ? a : b;
  const float equal = __builtin_signbitf(a) ? b : a;
  const float r = a == b ? equal : larger;
  return __builtin_isunordered(a, b) ? a + b : r;
}
__device__ __forceinline__ float wmin(float a, float b) {
  const float smaller = a < b ? a : b;
  const float equal = __builtin_signbitf(a) ? a : b;
  const float r = a == b ? equal : smaller;
  return __builtin_isunordered(a, b) ? a + b : r;
}

// the Cephes expf polynomial (S. L. Moshier's Cephes library) in the steps of kernels/kernel.ts:18-28
__device__ __forceinline__ float cephes_core(float x) {
  const float k = __builtin_rintf(x * 1.44269504088896341f);
  const float r = (x - k * 0.693359375f) - k * -2.12194440e-4f;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  const float e = (p * (r * r) + r) + 1.0f;
  return e * bits_f32((uint32_t)(trunc_sat(k) + 127) << 23);
}
// kernels/kernel.ts:15-29 fexp: 0 below -87, 88 above 88
__device__ __forceinline__ float fexp(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  return cephes_core(x);
}
// kernels/kernel.ts:33-45 vexp: x clamped to [-87, 88]
__device__ __forceinline__ float vexp(float x) { return cephes_core(wmin(wmax(x, -87.0f), 88.0f)); }

// kernels/kernel.ts:570-599 to_f16: round to nearest even; 65536 and above (and NaN) to infinity
__device__ __forceinline__ uint16_t to_f16(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const int32_t exponent = (int32_t)((bits >> 23) & 0xff) - 112;
  uint32_t mantissa = bits & 0x7fffffu;
  uint32_t result;
  if (exponent >= 31) {
    result = sign | 0x7c00u;
  } else if (exponent <= 0) {
    if (exponent < -10) {
      result = sign;
    } else {
      mantissa |= 0x800000u;
      const uint32_t shift = (uint32_t)(14 - exponent);
      const uint32_t rest = mantissa & ((1u << shift) - 1), middle = 1u << (shift - 1);
      uint32_t value = mantissa >> shift;
      if (rest > middle || (rest == middle && (value & 1))) value++;
      result = sign | value;
    }
  } else {
    const uint32_t rest = mantissa & 0x1fffu;
    uint32_t value = ((uint32_t)exponent << 10) | (mantissa >> 13);
    if (rest > 0x1000u || (rest == 0x1000u && (value & 1))) value++;
    result = sign | value;
  }
  return (uint16_t)result;
}

// kernels/kernel.ts:383-392 half: sign-extended bits shifted by 13, masked, times 2^112 (exact for every finite half)
__device__ __forceinline__ float from_f16(uint16_t h) {
  const int32_t bits = ((int32_t)(int16_t)h << 13) & (int32_t)0x8fffffff;
  return __int_as_float(bits) * 5.192296858534828e33f;
}

// ---- wave helpers (wave64) ----

// lane i ^ 1 (DPP quad_perm [1, 0, 3, 2]): a VALU operand, not a trip through the LDS unit as __shfl_xor is
__device__ __forceinline__ float dpp_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ int32_t dpp_xor1(int32_t v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true); }

// the largest over each half of the wave (32 lanes), order-free: xor 1 and xor 2 within quads, the mirrors within
// 8 and 16 lanes (DPP), then xor 16 (ds_swizzle); fmax ignores a NaN beside a number, as before
__device__ __forceinline__ float wave_max32(float v) {
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));
  v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  return v;
}

__device__ __forceinline__ float add32(float acc, const float4 v[8]) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    acc = acc + v[u].x;
    acc = acc + v[u].y;
    acc = acc + v[u].z;
    acc = acc + v[u].w;
  }
  return acc;
}

// the row stride (floats) of four ordered sums' values side by side in LDS: rows of q4 values 16-byte aligned and
// 64 bytes apart modulo 256, so that the four lanes' 16-byte reads of one step fall on distinct banks
__host__ __device__ constexpr int chain_rowstride(int q4) { return ((q4 + 63) & ~63) + 16; }

// acc + c[0] + c[1] + ... + c[n-1] in order (every add rounded), the values read from LDS 64 at a time: the second
// 32's reads fly while the first 32 are added. (No reads carried across iterations: a loop-carried set of registers
// makes the compiler copy it every iteration, which costs more than the latency it hides.) c 16-byte aligned.
template <int H = 8>
__device__ __forceinline__ float lds_chain_h(const float *c, int n, float acc) {
  const float4 *c4 = reinterpret_cast<const float4 *>(c);
  const int n4 = n >> 2;
  int i = 0;
  for (; i + 2 * H <= n4; i += 2 * H) {
    float4 a[H], b[H];
#pragma unroll
    for (int u = 0; u < H; ++u) a[u] = c4[i + u];
#pragma unroll
    for (int u = 0; u < H; ++u) b[u] = c4[i + H + u];
#pragma unroll
    for (int u = 0; u < H; ++u) {
      acc = acc + a[u].x;
      acc = acc + a[u].y;
      acc = acc + a[u].z;
      acc = acc + a[u].w;
    }
#pragma unroll
    for (int u = 0; u < H; ++u) {
      acc = acc + b[u].x;
      acc = acc + b[u].y;
      acc = acc + b[u].z;
      acc = acc + b[u].w;
    }
  }
  if (i + H <= n4) {
    float4 a[H];
#pragma unroll
    for (int u = 0; u < H; ++u) a[u] = c4[i + u];
#pragma unroll
    for (int u = 0; u < H; ++u) {
      acc = acc + a[u].x;
      acc = acc + a[u].y;
      acc = acc + a[u].z;
      acc = acc + a[u].w;
    }
    i += H;
  }
  for (; i < n4; ++i) {
    const float4 v = c4[i];
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  }
  for (int j = n4 << 2; j < n; ++j) acc = acc + c[j];
  return acc;
}
__device__ __forceinline__ float lds_chain(const float *c, int n, float acc) { return lds_chain_h<8>(c, n, acc); }

// An ordered sum run from registers by the 32 lanes of a half-wave: 0 + c[0] + c[1] + ... in order, every add
// rounded, over c = the sum's row of values (16-byte aligned), +0.0 from its count up to 32 * nseg (x + 0 is x for sums
// whose running values are never -0: they start at +0). Lane seg (0..31) of the half-wave is segment seg: in round
// s < nseg (nseg <= 32, the same in the whole wave) every lane adds its 32 values c[32 seg ..] to its running sum, and
// segment s's sum then goes to segment s + 1 (a DPP row shift inside a 16-lane row, a row broadcast from a row's last
// lane to the next row), so that lane s starts round s from the true running sum: the chain's adds come from registers
// (about 4.3 cycles an add against 8.5 for LDS reads in the chain). Returns the sum in the lane with seg == nseg - 1.
// Both half-waves of a wave run it together (each its own sum); the row broadcast writes only rows 1 and 3.
// nseg >= 1.
__device__ __forceinline__ float chain32_registers(const float *c, int nseg, int seg) {
  // lanes past the last segment read the first one (in the row; what they add is never used)
  const float4 *c4 = reinterpret_cast<const float4 *>(c + (seg < nseg ? seg : 0) * 32);
  float4 v[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) v[u] = c4[u];
  float acc = 0.0f;
  for (int s = 0; s < nseg; ++s) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc = acc + v[u].x;
      acc = acc + v[u].y;
      acc = acc + v[u].z;
      acc = acc + v[u].w;
    }
    const int src = __float_as_int(acc);
    const float moved = __int_as_float(s % 16 == 15 ? __builtin_amdgcn_update_dpp(src, src, 0x142, 0xA, 0xF, false)
                                                    : __builtin_amdgcn_update_dpp(src, src, 0x111, 0xF, 0xF, false));
    acc = seg == s + 1 ? moved : acc;
  }
  return acc;
}

// Four ordered sums of up to WAVE_CHAIN_MOST values each by two waves (chain32_registers with 32 rounds): thread
// t < 128 runs sum k = t / 32 over c_k = base + k * stride (+0.0 past its count up to WAVE_CHAIN_MOST), and thread
// 32 k + 31 returns it. 32 values a lane keep the register count low enough for two 1024-thread blocks a CU.
constexpr int WAVE_CHAIN_MOST = 1024;
__device__ __forceinline__ float chain4_registers(const float *base, int stride, int tid) {
  return chain32_registers(base + (tid >> 5) * stride, 32, tid & 31);
}

// a barrier of the workgroup over its LDS only: each wave's LDS accesses complete first (lgkmcnt), but not its global
// loads in flight, which a barrier with a workgroup fence of every address space waits for (on gfx9 one counter,
// vmcnt, holds a wave's loads and stores alike). No global store before it may be read after it by another wave.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// quantize_x of one group of 32, a half-wave (all 32 lanes present): amax (order-free), scale = f32(amax / qmax),
// inv = scale > 0 ? f32(1 / scale) : 0 (kernels/kernel.ts:129-156)
__device__ __forceinline__ void quantize_group(float v, int8_t *xq, float *xs, int j, int g, int32_t bias) {
  const float qmax = bias == 0 ? 127.0f : 63.0f;
  const float amax = wave_max32(__builtin_fabsf(v));
  const float scale = amax / qmax;
  const float inv = scale > 0 ? 1.0f / scale : 0.0f;
  xq[j] = quant_value(v, inv, bias);
  if ((threadIdx.x & 31) == 0) xs[g] = scale;
}

}  // namespace ple
