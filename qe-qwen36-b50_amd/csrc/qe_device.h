// Device-side building blocks shared by the MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qe_format.h"
#include "qe_synth.h"

#define QE_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------
// IQ4_NL decode: one dword of packed codes (bytes 4i..4i+3 of a block) gives
// elements 4i..4i+3 (low nibbles) and 16+4i..16+4i+3 (high nibbles) as int8x4.
// Two byte-permutes look the index up in codebook entries 0..7 and 8..15, a
// third picks per byte by the index's bit 3.
// ---------------------------------------------------------------------------
QE_DEV uint32_t nl4_lookup4(uint32_t idx /* 4 indices, one per byte, 0..15 */) {
    const uint32_t i7 = idx & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(QE_NL4_W1, QE_NL4_W0, i7); // entries 0..7
    const uint32_t b = __builtin_amdgcn_perm(QE_NL4_W3, QE_NL4_W2, i7); // entries 8..15
    const uint32_t sel = ((idx >> 1) & 0x04040404u) | 0x03020100u;     // bit 3 -> take b
    return __builtin_amdgcn_perm(b, a, sel);
}
QE_DEV void nl4_decode_dword(uint32_t q, uint32_t &lo, uint32_t &hi) {
    lo = nl4_lookup4(q & 0x0f0f0f0fu);
    hi = nl4_lookup4((q >> 4) & 0x0f0f0f0fu);
}
// Decoded 32-weight block: w[0..3] = elements 0..15, w[4..7] = elements 16..31,
// each dword holding 4 consecutive elements.
struct nl4_blk { uint32_t w[8]; };
QE_DEV nl4_blk nl4_decode_block(uint4 q) {
    nl4_blk r;
    nl4_decode_dword(q.x, r.w[0], r.w[4]);
    nl4_decode_dword(q.y, r.w[1], r.w[5]);
    nl4_decode_dword(q.z, r.w[2], r.w[6]);
    nl4_decode_dword(q.w, r.w[3], r.w[7]);
    return r;
}
// Exact int32 dot of a decoded block with 32 int8 activations (two uint4).
QE_DEV int nl4_block_dot(const nl4_blk &w, uint4 x0, uint4 x1) {
    int acc = 0;
    acc = __builtin_amdgcn_sdot4((int)w.w[0], (int)x0.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[1], (int)x0.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[2], (int)x0.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[3], (int)x0.w, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[4], (int)x1.x, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[5], (int)x1.y, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[6], (int)x1.z, acc, false);
    acc = __builtin_amdgcn_sdot4((int)w.w[7], (int)x1.w, acc, false);
    return acc;
}

QE_DEV float f16_bits_to_f32(uint16_t h) {
    _Float16 f;
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}

// ---------------------------------------------------------------------------
// cross-lane sums
// ---------------------------------------------------------------------------
// Canonical butterfly over 64 lanes (offsets 1,2,4,...,32): every lane ends
// with the pairwise-tree sum of the 64 lane values, the order the CPU checker
// restates for router rows and RMSNorm.
QE_DEV float wave_sum_canon(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}
// Sum within aligned groups of 16 lanes.
QE_DEV float sum16(float v) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}
QE_DEV float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// ---------------------------------------------------------------------------
// per-32 int8 quantisation of one block held as 32 floats by one lane, with
// the reference CPU semantics (engine/qe.cpp:687-703): d = amax/127,
// id = d>0 ? 1/d : 0, q = rint(x*id) saturated to int8.
// ---------------------------------------------------------------------------
QE_DEV int8_t quant_one(float x, float id) {
    float v = rintf(x * id);
    v = fminf(127.f, fmaxf(-128.f, v));
    return (int8_t)(int)v;
}
QE_DEV float quant_scale_inv(float amax, float &d) {
    d = amax / 127.f;
    return d > 0.f ? 1.f / d : 0.f;
}

QE_DEV float silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }
