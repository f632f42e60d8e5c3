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
// (v & 0x04040404) | 0x03020100.  VOP3 = true: one v_and_or_b32 (GFX9 VOP3
// takes no literal and one SGPR, so the mask rides in an SGPR and the byte
// ramp in a VGPR held across the loop); plain C: an and plus an or, no VGPR
// held (for kernels at their register limit).
template <bool VOP3> QE_DEV uint32_t nl4_merge_sel(uint32_t v) {
    if constexpr (VOP3) {
        uint32_t r;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(0x04040404u), "v"(0x03020100u));
        return r;
    } else {
        return (v & 0x04040404u) | 0x03020100u;
    }
}
// Both nibbles of 4 code bytes; the bit-3 selector comes straight from the
// code bytes (bits 3 and 7), without extracting the nibbles first.
template <bool VOP3 = false> QE_DEV void nl4_decode_dword(uint32_t q, uint32_t &lo, uint32_t &hi) {
    const uint32_t il = q & 0x07070707u, ih = (q >> 4) & 0x07070707u;
    const uint32_t sl = nl4_merge_sel<VOP3>(q >> 1), sh = nl4_merge_sel<VOP3>(q >> 5);
    lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(QE_NL4_W3, QE_NL4_W2, il), __builtin_amdgcn_perm(QE_NL4_W1, QE_NL4_W0, il), sl);
    hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(QE_NL4_W3, QE_NL4_W2, ih), __builtin_amdgcn_perm(QE_NL4_W1, QE_NL4_W0, ih), sh);
}
// Decoded 32-weight block: w[0..3] = elements 0..15, w[4..7] = elements 16..31,
// each dword holding 4 consecutive elements.
struct nl4_blk { uint32_t w[8]; };
template <bool VOP3 = false> QE_DEV nl4_blk nl4_decode_block(uint4 q) {
    nl4_blk r;
    nl4_decode_dword<VOP3>(q.x, r.w[0], r.w[4]);
    nl4_decode_dword<VOP3>(q.y, r.w[1], r.w[5]);
    nl4_decode_dword<VOP3>(q.z, r.w[2], r.w[6]);
    nl4_decode_dword<VOP3>(q.w, r.w[3], r.w[7]);
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
// Lane exchanges are single VALU ops: DPP within 16-lane rows and the gfx950
// row swaps across rows (an __shfl_xor is a ds_bpermute, an LDS round trip).
//   QE_DPP_XOR1 / XOR2: quad_perm [1,0,3,2] / [2,3,0,1];
//   QE_DPP_HMIRROR: lane i <-> 7 - i within 8;  QE_DPP_MIRROR: i <-> 15 - i within 16.
// After a reduction over aligned groups of g lanes every lane of a group holds
// the group's value, so a mirror pairs each lane with the other half's value
// exactly as the xor butterfly would.
#define QE_DPP_XOR1 0xB1
#define QE_DPP_XOR2 0x4E
#define QE_DPP_HMIRROR 0x141
#define QE_DPP_MIRROR 0x140
template <int CTRL> QE_DEV unsigned dpp_u(unsigned v) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL> QE_DEV float dpp_f(float v) { return __uint_as_float(dpp_u<CTRL>(__float_as_uint(v))); }
// Rows of 16 lanes r0..r3: a = [r0 r0 r2 r2], b = [r1 r1 r3 r3] (16-lane swap)
// or a = [r0 r1 r0 r1], b = [r2 r3 r2 r3] (32-lane swap) of v.
QE_DEV void rows16(unsigned v, unsigned &a, unsigned &b) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = s[0];
    b = s[1];
}
QE_DEV void rows32(unsigned v, unsigned &a, unsigned &b) {
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = s[0];
    b = s[1];
}
// Sum within aligned groups of 16 lanes, pairwise tree (lanes (i, i^1) first).
QE_DEV float sum16(float v) {
    v = v + dpp_f<QE_DPP_XOR1>(v);
    v = v + dpp_f<QE_DPP_XOR2>(v);
    v = v + dpp_f<QE_DPP_HMIRROR>(v);
    v = v + dpp_f<QE_DPP_MIRROR>(v);
    return v;
}
// Rows of a 16-uniform value: [r0 + r1, r0 + r1, r2 + r3, r2 + r3] / sum of all four.
QE_DEV float add_rows16(float v) {
    unsigned a, b;
    rows16(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}
QE_DEV float add_rows32(float v) {
    unsigned a, b;
    rows32(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}
// Canonical pairwise tree over 64 lanes (lane pairs, then pairs of pairs, ...):
// every lane ends with the tree sum of the 64 lane values, the order the CPU
// checker restates for router rows and RMSNorm.
QE_DEV float wave_sum_canon(float v) { return add_rows32(add_rows16(sum16(v))); }
QE_DEV float max16(float v) {
    v = fmaxf(v, dpp_f<QE_DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<QE_DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<QE_DPP_HMIRROR>(v));
    return fmaxf(v, dpp_f<QE_DPP_MIRROR>(v));
}
// |v| maximum within aligned groups of 16 lanes, on the bit patterns: for floats
// >= 0 the u32 order is the float order, and an unsigned maximum needs no NaN
// canonicalisation, so each step is one v_max_u32 with a DPP source
QE_DEV float max16_abs(float v) {
    unsigned u = __float_as_uint(v) & 0x7fffffffu;
    u = max(u, dpp_u<QE_DPP_XOR1>(u));
    u = max(u, dpp_u<QE_DPP_XOR2>(u));
    u = max(u, dpp_u<QE_DPP_HMIRROR>(u));
    return __uint_as_float(max(u, dpp_u<QE_DPP_MIRROR>(u)));
}
// maximum within aligned groups of 32 lanes
QE_DEV float max32(float v) {
    unsigned a, b;
    rows16(__float_as_uint(max16(v)), a, b);
    return fmaxf(__uint_as_float(a), __uint_as_float(b));
}
// u32 maximum over the wave; the DPP moves use bound_ctrl (every source lane
// exists in these patterns) so they can fold into the v_max_u32 that uses them.
template <int CTRL> QE_DEV unsigned dpp_ub(unsigned v) {
    return (unsigned)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}
QE_DEV unsigned umax32(unsigned a, unsigned b) { return a > b ? a : b; }
QE_DEV unsigned wave_max_u32(unsigned v) {
    v = umax32(v, dpp_ub<QE_DPP_XOR1>(v));
    v = umax32(v, dpp_ub<QE_DPP_XOR2>(v));
    v = umax32(v, dpp_ub<QE_DPP_HMIRROR>(v));
    v = umax32(v, dpp_ub<QE_DPP_MIRROR>(v));
    unsigned a, b;
    rows16(v, a, b);
    v = umax32(a, b);
    rows32(v, a, b);
    return umax32(a, b);
}
QE_DEV unsigned umin32(unsigned a, unsigned b) { return a < b ? a : b; }
// Bitonic sort of 32 lanes (each half of the wave on its own), descending by
// the 64-bit key (hi, lo), every comparator pointing the same way: for blocks
// k = 2, 4, .., 32, lane i meets its mirror i ^ (k - 1) in the block, then
// i ^ j for j = k/4 .. 1, and the lower lane of each pair keeps the larger
// key.  Partners come by DPP (quad_perm, row mirrors, row_ror:8 for xor 8,
// row_shr/shl:4 for xor 4) and, for the 32-lane mirror, a 16-lane row swap.
QE_DEV void cx64(uint32_t &hi, uint32_t &lo, uint32_t phi, uint32_t plo, bool lower) {
    const uint64_t k = ((uint64_t)hi << 32) | lo, p = ((uint64_t)phi << 32) | plo;
    if (lower == (p > k)) {
        hi = phi;
        lo = plo;
    }
}
QE_DEV void sort32_desc_u64(uint32_t &hi, uint32_t &lo, int lane) {
    auto xor1 = [&]() { cx64(hi, lo, dpp_u<QE_DPP_XOR1>(hi), dpp_u<QE_DPP_XOR1>(lo), !(lane & 1)); };
    auto xor2 = [&]() { cx64(hi, lo, dpp_u<QE_DPP_XOR2>(hi), dpp_u<QE_DPP_XOR2>(lo), !(lane & 2)); };
    auto xor4 = [&]() { // row_shr:4 (from lane i - 4) where bit 2 is set, row_shl:4 (from i + 4) where clear
        const bool up = lane & 4;
        const uint32_t rh = dpp_u<0x114>(hi), lh = dpp_u<0x104>(hi); // both, then a select:
        const uint32_t rl = dpp_u<0x114>(lo), ll = dpp_u<0x104>(lo); // DPP does not run under a branch
        cx64(hi, lo, up ? rh : lh, up ? rl : ll, !up);
    };
    xor1();                                                                           // k = 2
    cx64(hi, lo, dpp_u<0x1B>(hi), dpp_u<0x1B>(lo), !(lane & 2));                      // k = 4: quad_perm [3,2,1,0]
    xor1();
    cx64(hi, lo, dpp_u<QE_DPP_HMIRROR>(hi), dpp_u<QE_DPP_HMIRROR>(lo), !(lane & 4));  // k = 8
    xor2();
    xor1();
    cx64(hi, lo, dpp_u<QE_DPP_MIRROR>(hi), dpp_u<QE_DPP_MIRROR>(lo), !(lane & 8));    // k = 16
    xor4();
    xor2();
    xor1();
    {   // k = 32: the mirror in the other 16-lane row of the pair
        unsigned ah, bh, al, bl;
        rows16(dpp_u<QE_DPP_MIRROR>(hi), ah, bh);
        rows16(dpp_u<QE_DPP_MIRROR>(lo), al, bl);
        const bool r1 = lane & 16;
        cx64(hi, lo, r1 ? ah : bh, r1 ? al : bl, !r1);
    }
    cx64(hi, lo, dpp_u<0x128>(hi), dpp_u<0x128>(lo), !(lane & 8));                  // row_ror:8 = xor 8
    xor4();
    xor2();
    xor1();
}

// The same network on 32-bit keys (each step a max, a min and a select).
QE_DEV void cx32(uint32_t &k, uint32_t p, bool lower) {
    const uint32_t mx = k > p ? k : p, mn = k > p ? p : k;
    k = lower ? mx : mn;
}
QE_DEV void sort32_desc_u32(uint32_t &k, int lane) {
    auto xor1 = [&]() { cx32(k, dpp_u<QE_DPP_XOR1>(k), !(lane & 1)); };
    auto xor2 = [&]() { cx32(k, dpp_u<QE_DPP_XOR2>(k), !(lane & 2)); };
    auto xor4 = [&]() {
        const bool up = lane & 4;
        const uint32_t r = dpp_u<0x114>(k), l = dpp_u<0x104>(k);
        cx32(k, up ? r : l, !up);
    };
    xor1();                                              // k = 2
    cx32(k, dpp_u<0x1B>(k), !(lane & 2));                // k = 4
    xor1();
    cx32(k, dpp_u<QE_DPP_HMIRROR>(k), !(lane & 4));      // k = 8
    xor2();
    xor1();
    cx32(k, dpp_u<QE_DPP_MIRROR>(k), !(lane & 8));       // k = 16
    xor4();
    xor2();
    xor1();
    {   // k = 32
        unsigned a, b;
        rows16(dpp_u<QE_DPP_MIRROR>(k), a, b);
        const bool r1 = lane & 16;
        cx32(k, r1 ? a : b, !r1);
    }
    cx32(k, dpp_u<0x128>(k), !(lane & 8));
    xor4();
    xor2();
    xor1();
}

// Lane 63 - i's value (the mirror across the wave): the row mirror of lane
// i ^ 32, then of lane i ^ 48.  And lane i ^ 16's value.
QE_DEV uint32_t lane_mirror64(uint32_t v, int lane) {
    unsigned a, b, c, d;
    rows32(dpp_u<QE_DPP_MIRROR>(v), a, b);
    rows16((lane & 32) ? a : b, c, d);
    return (lane & 16) ? c : d;
}
QE_DEV uint32_t lane_xor16(uint32_t v, int lane) {
    unsigned a, b;
    rows16(v, a, b);
    return (lane & 16) ? a : b;
}
// The last stage (k = 64) of the bitonic network: with lanes 0..31 and 32..63
// each sorted descending (sort32_desc_*), the wave becomes one descending run.
QE_DEV void merge64_desc_u32(uint32_t &k, int lane) {
    cx32(k, lane_mirror64(k, lane), !(lane & 32));
    cx32(k, lane_xor16(k, lane), !(lane & 16));
    cx32(k, dpp_u<0x128>(k), !(lane & 8)); // row_ror:8 = xor 8
    const bool up = lane & 4;
    const uint32_t r = dpp_u<0x114>(k), l = dpp_u<0x104>(k);
    cx32(k, up ? r : l, !up);
    cx32(k, dpp_u<QE_DPP_XOR2>(k), !(lane & 2));
    cx32(k, dpp_u<QE_DPP_XOR1>(k), !(lane & 1));
}
QE_DEV void merge64_desc_u64(uint32_t &hi, uint32_t &lo, int lane) {
    cx64(hi, lo, lane_mirror64(hi, lane), lane_mirror64(lo, lane), !(lane & 32));
    cx64(hi, lo, lane_xor16(hi, lane), lane_xor16(lo, lane), !(lane & 16));
    cx64(hi, lo, dpp_u<0x128>(hi), dpp_u<0x128>(lo), !(lane & 8));
    const bool up = lane & 4;
    const uint32_t rh = dpp_u<0x114>(hi), lh = dpp_u<0x104>(hi);
    const uint32_t rl = dpp_u<0x114>(lo), ll = dpp_u<0x104>(lo);
    cx64(hi, lo, up ? rh : lh, up ? rl : ll, !up);
    cx64(hi, lo, dpp_u<QE_DPP_XOR2>(hi), dpp_u<QE_DPP_XOR2>(lo), !(lane & 2));
    cx64(hi, lo, dpp_u<QE_DPP_XOR1>(hi), dpp_u<QE_DPP_XOR1>(lo), !(lane & 1));
}

QE_DEV unsigned wave_min_u32(unsigned v) {
    v = umin32(v, dpp_ub<QE_DPP_XOR1>(v));
    v = umin32(v, dpp_ub<QE_DPP_XOR2>(v));
    v = umin32(v, dpp_ub<QE_DPP_HMIRROR>(v));
    v = umin32(v, dpp_ub<QE_DPP_MIRROR>(v));
    unsigned a, b;
    rows16(v, a, b);
    v = umin32(a, b);
    rows32(v, a, b);
    return umin32(a, b);
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

// ===========================================================================
// top-8 of one token by one wave (engine/qe.cpp:1454-1483 semantics):
// maximum logit first; ties go to the smaller (e % 16, e / 16), the order the
// reference's 16-lane reduction produces.  Lane l holds e = l + 64 j.
// ===========================================================================
// Order-preserving u32 image of a float (-0 folded onto +0 by the caller).
QE_DEV unsigned f2ord(float v) {
    const unsigned u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
QE_DEV float ord2f(unsigned o) { return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o); }

// Weights and shared gate of a selection: lane k < 8 holds the k-th selected
// logit `mine` and its expert; sel0 is the largest.  w_k = exp(l_k - l_0) /
// sum_j exp(l_j - l_0), the sum in k order; shg = sigmoid(logit 256).
QE_DEV void topk_finish(float mine, int myid, float sel0, float lg_sh, int lane, int32_t *ids, float *wts, float *shg) {
    const float ex = expf(mine - sel0);
    float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), 0));
#pragma unroll
    for (int k = 1; k < QE_K_USED; ++k) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), k));
    if (lane < QE_K_USED) {
        ids[lane] = myid;
        wts[lane] = ex / s;
    }
    if (lane == QE_K_USED) *shg = 1.f / (1.f + expf(-lg_sh));
}

// v[j] = logit of expert lane + 64 j; lg_sh = logit 256 (shared-expert gate).
// Each round: one wave max of the values (as order-preserving u32, -0 folded
// onto +0, so equal logits compare equal as in the reference), then one wave
// min of the tie-break keys (e % 16) * 16 + e / 16 over the slots holding it.  The softmax weights run one per lane;
// their sum keeps the reference's order k = 0..7.
// Returns, in lane k < 8, the k-th selected expert.
QE_DEV int wave_topk_vals(const float v_in[4], float lg_sh, int lane, int32_t *ids, float *wts, float *shg) {
    unsigned v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = f2ord(v_in[j] + 0.0f);
    float sel[QE_K_USED];
    int id[QE_K_USED];
    // tie-break key of slot j: (e % 16) * 16 + e / 16 with e = lane + 64 j
    const unsigned key0 = (unsigned)((lane & 15) * 16 + (lane >> 4));
#pragma unroll
    for (int k = 0; k < QE_K_USED; ++k) {
        const unsigned m = wave_max_u32(umax32(umax32(v[0], v[1]), umax32(v[2], v[3])));
        // smallest key among the holders of m, by a second wave reduction
        unsigned ck = 0xffffu;
#pragma unroll
        for (int j = 3; j >= 0; --j) ck = v[j] == m ? key0 + 4 * j : ck;
        const unsigned kmin = wave_min_u32(ck);
        sel[k] = ord2f(m);
        id[k] = (int)(((kmin & 15u) << 4) | ((kmin >> 4) & 15u)); // in 0..255 whatever the data
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (key0 + 4 * j == kmin) v[j] = 0u; // below every ordered float
    }
    float mine = sel[0];
    int myid = id[0];
#pragma unroll
    for (int k = 1; k < QE_K_USED; ++k)
        if (lane == k) { mine = sel[k]; myid = id[k]; }
    topk_finish(mine, myid, sel[0], lg_sh, lane, ids, wts, shg);
    return myid;
}

// The same selection, usually in fewer steps: each lane's maximum over its
// four, then over groups of 8 lanes, gives eight maxima of distinct experts;
// the smallest of them bounds the 8th largest logit from below, so the experts
// at or above it (about 20 of 256; more than 32 for 7 % of random tokens, more
// than 64 for 0.05 %) hold the top 8.  Up to 64 of them go one per lane through `sk` (64 words of
// LDS) as 64-bit keys {ordered value, 0xffff - tie key} and are sorted in
// registers (the 64-wide stage only when more than 32 survive); lanes 0..7
// then hold the selection in the reference's order.  More survivors (many
// equal logits) take the rounds of wave_topk_vals.  Returns, in lane k < 8,
// the k-th selected expert.
QE_DEV int wave_topk_sorted(const float v_in[4], float lg_sh, int lane, uint64_t *sk, int32_t *ids, float *wts,
                            float *shg) {
    unsigned v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = f2ord(v_in[j] + 0.0f);
    unsigned g = umax32(umax32(v[0], v[1]), umax32(v[2], v[3]));
    g = umax32(g, dpp_ub<QE_DPP_XOR1>(g));
    g = umax32(g, dpp_ub<QE_DPP_XOR2>(g));
    g = umax32(g, dpp_ub<QE_DPP_HMIRROR>(g)); // maximum of 32 experts (8 lanes)
    g = umin32(g, dpp_ub<QE_DPP_MIRROR>(g));
    unsigned ra, rb;
    rows16(g, ra, rb);
    g = umin32(ra, rb);
    rows32(g, ra, rb);
    g = umin32(ra, rb); // the smallest of the eight
    int S = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool sv = v[j] >= g;
        const unsigned long long bal = __ballot(sv);
        const int pos = S + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
        const int e = lane + 64 * j;
        if (sv && pos < 64) sk[pos] = ((uint64_t)v[j] << 32) | (0xffffu - (unsigned)((e & 15) * 16 + (e >> 4)));
        S += (int)__popcll(bal);
    }
    if (S > 64) return wave_topk_vals(v_in, lg_sh, lane, ids, wts, shg);
    const uint64_t ki = lane < S ? sk[lane] : 0ull; // real keys are never 0
    uint32_t khi = (uint32_t)(ki >> 32), klo = (uint32_t)ki;
    sort32_desc_u64(khi, klo, lane);
    if (S > 32) merge64_desc_u64(khi, klo, lane);
    const unsigned tk = 0xffffu - (klo & 0xffffu); // (e % 16) * 16 + e / 16
    const int myid = (int)(((tk & 15u) << 4) | ((tk >> 4) & 15u));
    const float sel0 = ord2f((unsigned)__builtin_amdgcn_readfirstlane(khi));
    topk_finish(ord2f(khi), myid, sel0, lg_sh, lane, ids, wts, shg);
    return myid;
}
// Canonical RMSNorm sum of squares of a 2048-vector: 256 groups of 8
// contiguous elements, each an fma chain from 0 in index order, combined by the
// pairwise tree over the groups (adjacent pairs first).  A lane holding the 32
// elements [32c, 32c+32) forms groups 4c..4c+3 and the first two tree levels;
// wave_sum_canon over the 64 lanes is the rest of the tree.  (Groups of 8 are
// what one decode workgroup produces, so its partial travels with its rows.)
QE_DEV float sumsq_group8(const float *v) {
    float g = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) g = fmaf(v[i], v[i], g);
    return g;
}
QE_DEV float sumsq_lane32(const float v[32]) {
    return (sumsq_group8(v) + sumsq_group8(v + 8)) + (sumsq_group8(v + 16) + sumsq_group8(v + 24));
}

// One canonical normalisation of a 2048-vector by one wave.  Lane c owns the
// 32 contiguous elements [32c, 32c+32) in v[]; on return v holds xn.
QE_DEV void wave_norm_chunk(float v[32], const float *post_norm, int lane) {
    if (!post_norm) return;
    const float ss = wave_sum_canon(sumsq_lane32(v));
    const float inv = 1.0f / sqrtf(ss / (float)QE_D + QE_RMS_EPS);
    const float4 *wr = (const float4 *)(post_norm + lane * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 w = wr[i];
        v[4 * i + 0] = (v[4 * i + 0] * inv) * w.x;
        v[4 * i + 1] = (v[4 * i + 1] * inv) * w.y;
        v[4 * i + 2] = (v[4 * i + 2] * inv) * w.z;
        v[4 * i + 3] = (v[4 * i + 3] * inv) * w.w;
    }
}

// Quantise the 32 values a lane holds (one block) and store int8 + scale.
QE_DEV void lane_quant_store(const float v[32], int8_t *q_out, float *s_out) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    float d;
    const float id = quant_scale_inv(amax, d);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t x = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) x |= (uint32_t)(uint8_t)quant_one(v[4 * i + j], id) << (8 * j);
        w[i] = x;
    }
    ((uint4 *)q_out)[0] = make_uint4(w[0], w[1], w[2], w[3]);
    ((uint4 *)q_out)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *s_out = d;
}

// Operand layout of int8 activation rows for the prefill MFMA GEMMs: per pair
// of 32-blocks (2q, 2q+1), 64 bytes = 4 groups g of 16 bytes; group g holds
// 8 bytes of block 2q then 8 of block 2q+1, each run being elements
// 4g..4g+3 followed by 16+4g..16+4g+3 of its block.
QE_HD int qe_opnd_off(int k) {
    const int b = k >> 5, e = k & 31;
    return (b >> 1) * 64 + ((e & 15) >> 2) * 16 + (b & 1) * 8 + (e >> 4) * 4 + (e & 3);
}
// quantise block b = lane of a row (as lane_quant_store) into the operand layout
QE_DEV void lane_quant_store_opnd(const float v[32], int8_t *row, int b, float *s_out) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    float d;
    const float id = quant_scale_inv(amax, d);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t x = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) x |= (uint32_t)(uint8_t)quant_one(v[4 * i + j], id) << (8 * j);
        w[i] = x; // elements 4i..4i+3
    }
    int8_t *dst = row + (b >> 1) * 64 + (b & 1) * 8;
#pragma unroll
    for (int g = 0; g < 4; ++g) *(uint2 *)(dst + 16 * g) = make_uint2(w[g], w[4 + g]);
    *s_out = d;
}

// fp32 activations for the fp16 matrix cores: a = a_hi + a_lo with
// a_hi = fp16(a), a_lo = fp16(a - a_hi) (the difference is exact in fp32), so
// a_hi + a_lo carries ~22 significant bits for |a| < 65504.
// Rows are stored in the operand order of v_mfma_f32_32x32x16_f16, 32 rows per
// tile: per 32-block b, four 1 KB chunks q of 64 lanes x 16 B, where lane
// l = r + 32 kh (row r of the tile) holds, for q = 0..3: hi of block elements
// 16 kh + 0..7, hi of 16 kh + 8..15, lo of 16 kh + 0..7, lo of 16 kh + 8..15.
// One dwordx4 load per lane and chunk reads 1 KB contiguous.  Byte offset of
// the hi half of element k of row `row` (K elements per row); lo is 2048 B on.
QE_HD size_t qe_hl_off(int K, int row, int k) {
    const int e = k & 31;
    return ((((size_t)(row >> 5) * (K / 32) + (k >> 5)) * 4 + ((e >> 3) & 1)) * 64 + (row & 31) + 32 * (e >> 4)) * 16 +
           2 * (e & 7);
}
#define QE_HL_LO 2048
QE_DEV uint32_t pack_h2(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

QE_DEV void load32(const float *p, float v[32]) {
    const float4 *q = (const float4 *)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = q[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}
QE_DEV void unpack_i8x32(uint4 a, uint4 b, float w[32]) {
    const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) w[4 * i + j] = (float)(int8_t)((d[i] >> (8 * j)) & 0xff);
}

