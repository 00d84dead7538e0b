// attention.hpp — what the decode (attention.hip) and the prompt (attention_tokens.hip) attention kernels share: the
// tile and grouping constants, the cache readers (float32 or float16, read as kernels/kernel.ts:383-392 reads them)
// and the prompt kernels' launchers.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace ple {

constexpr int TILE = 64;   // positions a block of (A)
constexpr int MAXMUL = 8;  // query heads a kv head at most
constexpr int DECODE_TOKENS = 8;  // up to this many tokens a launch runs the decode kernels (attention.hip)

template <bool HALF>
__device__ __forceinline__ float4 cache4(const void *c, int64_t i) {  // four values from element i (i % 4 == 0)
  if constexpr (HALF) {
    const uint2 h = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(c) + i);
    return make_float4(from_f16((uint16_t)(h.x & 0xffff)), from_f16((uint16_t)(h.x >> 16)),
                       from_f16((uint16_t)(h.y & 0xffff)), from_f16((uint16_t)(h.y >> 16)));
  } else {
    return *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(c) + i);
  }
}
template <bool HALF>
__device__ __forceinline__ float cache1(const void *c, int64_t i) {
  if constexpr (HALF) return from_f16(reinterpret_cast<const uint16_t *>(c)[i]);
  else return reinterpret_cast<const float *>(c)[i];
}

// the launch's first position: from device memory in a replayed decode step (where a.pos0 only bounds it)
__device__ __forceinline__ int first_position(const AttnArgs &a) { return a.dpos ? *a.dpos : a.pos0; }

constexpr int ALDS = 160 * 1024 - 256;  // LDS a block may take (gfx950: 160 KiB a workgroup), less the static part

// the prompt's kernels (attention_tokens.hip): the scores of many tokens (scores_tokens_kernel), and the separate
// softmax (softmax_kernel) and weighted values (pv_tokens_kernel) that prompt blocks and contexts past the decode
// kernels' LDS take; the LDS a (token, head) of count positions takes in softmax_kernel
hipError_t launch_scores_tokens(const AttnArgs &a, hipStream_t s);
hipError_t launch_softmax_pv(const AttnArgs &a, hipStream_t s);
size_t softmax_lds(int count);
size_t softmax4_lds(int count);

}  // namespace ple
