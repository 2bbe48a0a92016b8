// Buffer-load helpers of the weight-streaming kernels (the skinny grouped
// GEMM and the fused decode MoE's down projection).
#pragma once

#include "qmoe_common.h"

namespace qmoe_stream {

// 64 bytes of one operand's step: up to 4 x 16 B chunks
struct Frag {
  uint4 v[4];
};

// Operands are read with buffer loads: a wave-uniform resource (base and
// extent in SGPRs), a 32-bit per-lane offset fixed for the whole K loop, and
// the step's byte offset as a scalar. This keeps one VGPR per stream instead
// of a 64-bit address per load; the host keeps every operand below 2 GiB.
using rsrc_t = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes >= 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// A lane offset with this bit set is past every buffer's extent (the host
// keeps operands below 2 GiB, and lane offsets below 2 GiB have the bit
// clear): the load returns zeros and makes no memory request. The bit goes in
// the per-lane offset, which the range check always covers; the scalar step
// offset stays a valid one.
constexpr uint32_t kOob = 0x80000000u;

// NB/16 weight chunks of one step: 16 B at voff + j*64 (the lane's column of
// 64 B segment j of its load row)
template <int NB, int AUX = 0>
__device__ __forceinline__ void ldw_seg(Frag& f, rsrc_t r, uint32_t voff, uint32_t soff) {
#pragma unroll
  for (int j = 0; j < NB / 16; ++j) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + j * 64, soff, AUX);
    f.v[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// Weight loads put row (l >> 2), column (l & 3) of a 64 B segment in lane l,
// so the 4 lanes of each 64 B piece are adjacent (the load is coalesced);
// the MFMA wants row (l & 15), k-group (l >> 4) in lane l. `src` is the
// byte address of lane 4*(l & 15) + (l >> 4).
template <int NB>
__device__ __forceinline__ void permute_w(Frag& f, int src) {
#pragma unroll
  for (int j = 0; j < NB / 16; ++j) {
    f.v[j].x = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)f.v[j].x);
    f.v[j].y = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)f.v[j].y);
    f.v[j].z = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)f.v[j].z);
    f.v[j].w = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)f.v[j].w);
  }
}

__device__ __forceinline__ float ldb_f32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

__device__ __forceinline__ i32x8 as_i32x8(const Frag& f) {
  i32x8 r;
  r[0] = f.v[0].x; r[1] = f.v[0].y; r[2] = f.v[0].z; r[3] = f.v[0].w;
  r[4] = f.v[1].x; r[5] = f.v[1].y; r[6] = f.v[1].z; r[7] = f.v[1].w;
  return r;
}

}  // namespace qmoe_stream
