// Prefill (T > 8) matrix-core kernels: the routed experts as int8 MFMA grouped
// GEMMs (Engine::moe_round_xmx and moe_xmx, engine/qe.cpp:2103-2154 and
// :369-436, redesigned for CDNA4), the router tiles and the Q8 shared expert.
//
// Exactness: the reference CPU path multiplies int8 activations by IQ4_NL
// codebook values exactly per 32-block and applies fp32 block scales after
// (engine/qe.cpp:704-741).  v_mfma_i32_16x16x32_i8 consumes one 32-element
// block per instruction, so every block dot is an exact int32, and the fp32
// epilogue applies xs[m][b] * dw[n][b] per block: results agree with the CPU
// path to fp32 rounding.  (Scaled fp16/bf16 operands would not: the h
// quantisation downstream turns 1e-4 relative noise into >1e-3 output error.)
//
// Work item: (expert e, up to 64 of its pairs in dispatch order) x row group.
//   gate/up epilogue: h = silu(g)*u, quantised per 32-block (the quant_x step
//   of engine/qe.cpp:2078-2081), stored int8 in the operand layout + fp32 scales;
//   down epilogue: yp[p][n] = w_p * y.
#include "qe_kernels.h"

typedef _Float16 qe_half8 __attribute__((ext_vector_type(8)));

// int32 -> fp32 without a conversion: the float with bits 0x4B400000 + P is
// 3 * 2^22 + P exactly for |P| < 2^22 (the binade [2^23, 2^24) has ulp 1).
#define QE_I2F_MAGIC_BITS 0x4B400000
#define QE_I2F_MAGIC 12582912.0f


// fp16 of small integers: half(0x6400 | u) = 1024 + u for u in 0..1023, so a
// biased byte u = v + 128 becomes v exactly after subtracting 1152.
QE_DEV uint32_t bias_bytes_to_h2(uint32_t u4, int hi_pair) {
    // bytes (u0,u1) or (u2,u3) of u4 -> two halves 0x64uu
    return __builtin_amdgcn_perm(0x64646464u, u4, hi_pair ? 0x07030702u : 0x07010700u);
}
QE_DEV void biased4_to_half4(uint32_t u4, uint32_t &h01, uint32_t &h23) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    uint32_t a = bias_bytes_to_h2(u4, 0), b = bias_bytes_to_h2(u4, 1);
    h2 ha = __builtin_bit_cast(h2, a) + off, hb = __builtin_bit_cast(h2, b) + off;
    h01 = __builtin_bit_cast(uint32_t, ha);
    h23 = __builtin_bit_cast(uint32_t, hb);
}
// 8 int8 (two dwords) -> 8 fp16
QE_DEV qe_half8 i8x8_to_half8(uint32_t lo, uint32_t hi) {
    uint32_t h[4];
    biased4_to_half4(lo ^ 0x80808080u, h[0], h[1]);
    biased4_to_half4(hi ^ 0x80808080u, h[2], h[3]);
    return __builtin_bit_cast(qe_half8, make_uint4(h[0], h[1], h[2], h[3]));
}
// 4 NL4 indices (one per byte) -> 4 codebook values as biased bytes (v + 128)
QE_DEV uint32_t nl4_lookup4_biased(uint32_t idx) { return nl4_lookup4(idx) ^ 0x80808080u; }

struct GemmTileArgs {
    const uint8_t *arena;      // layer's 256 expert blobs
    const int8_t *aq;          // int8 activations in the operand layout (qe_opnd_off), row = token or pair
    int a_bytes;               // size of aq in bytes
    const float *as;           // their fp32 block scales
    int a_row_div;             // pair -> activation row: p / a_row_div (8 for tokens, 1 for pairs)
    const int32_t *pairs;
    const int4 *items;         // (expert, first pair, count <= QE_MFMA_MC)
    const int32_t *n_items;
    const float *wts;          // pair weights (down)
    int8_t *hq; float *hs;     // gate/up output: quantised h (operand layout) + block scales
    float *yp;                 // down output
    int dn_rgw;                // down: row groups of 128 output rows per workgroup (1, 2 or 4)
    int32_t *item_done;        // fused gate/up + down launch: gate/up workgroups done per item (else nullptr)
    unsigned *err;             // fused launch: where a down workgroup's wait that gave up is recorded
    unsigned err_val;          //   (the value it stores there)
    int spin_cap;              //   and the reads a wait may take
    int wait_extra;            //   test hook: more gate/up workgroups than the item has (0 in use)
};

// Stores and loads through to the device coherence point (sc1): the h of a gate/up
// workgroup is read by down workgroups of the same launch in the fused form, on
// whatever XCD they run, with no L2 write-back or invalidation between them.
typedef unsigned qe_st_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned qe_st_u32x2 __attribute__((ext_vector_type(2)));
QE_DEV void st_sc1(void *p, uint4 v) {
    const qe_st_u32x4 w = {v.x, v.y, v.z, v.w};
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}
QE_DEV void st_sc1(void *p, uint2 v) {
    const qe_st_u32x2 w = {v.x, v.y};
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}
QE_DEV void st_sc1(void *p, float v) { asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory"); }
QE_DEV float4 ld_sc1_f4(const void *p) {
    qe_st_u32x4 w;
    asm volatile("global_load_dwordx4 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(w) : "v"(p) : "memory");
    return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
}

// v_mfma_i32_16x16x32_i8 with one 32-element block per instruction keeps the
// block dot an exact int32; lane l supplies k = 8 (l / 16) + 0..7 of row / column
// l % 16 and receives D[4 (l / 16) + i][l % 16].  The 8 k of group g are the
// block elements 4g..4g+3 and 16+4g..16+4g+3, i.e. both nibbles of code bytes
// 4g..4g+3, so a lane's B operand is one dword of codes and its A operand one
// 8-byte run of the operand layout.
//
// Wave = 16 NC weight rows (NC column groups of 16) x NT 16-pair tiles, streaming
// K in turns of 8 blocks.  Codes arrive 16 bytes per lane: lane (n, g) loads
// block 4Q+g of its row, four 16-lane rows of the wave cover a quad of blocks,
// and a 4x4 transpose over the rows (v_permlane32_swap, v_permlane16_swap)
// hands lane (n, g) dword g of each block of the quad.  The code ring holds two
// quads; loads are never predicated (the last refills wrap to the first blocks)
// and each refill takes an offset that depends on the last read of its slot,
// so it is issued 8 blocks ahead of its use into the slot's own registers.
// The four waves of a workgroup share the item's pairs: each quad's activations
// (128 bytes of K per pair) and block scales, and the weight scales of the
// workgroup's rows, are loaded once per workgroup into a double-buffered LDS
// stage (issued a quad ahead, stored and published by one barrier at the end of
// the quad), and every wave reads its A operands from there.
typedef unsigned qe_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned qe_u32x4 __attribute__((ext_vector_type(4)));

// rows r of d[0..3] -> d[j] row r = d[r] row j (16-lane rows of the wave)
QE_DEV void transpose_rows4(uint32_t d[4]) {
    qe_u32x2 x = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
    qe_u32x2 y = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
    const qe_u32x2 u = __builtin_amdgcn_permlane16_swap(x.x, y.x, false, false);
    const qe_u32x2 v = __builtin_amdgcn_permlane16_swap(x.y, y.y, false, false);
    d[0] = u.x; d[1] = u.y; d[2] = v.x; d[3] = v.y;
}

// LDS of one (NC, NT) tile, in bytes from the start of ExpertSmem::raw:
//   weight scales of the workgroup's rows, whole K: fp16 [block][wave][n][group];
//   two stages of the item's activations for one quad (4 blocks): [pair][128 bytes],
//     the 16-byte chunk q of pair m stored at chunk q ^ (m / 2 % 8) -- the sixteen
//     rows a lane group reads in one instruction fall in sixteen different bank
//     groups; a stage also holds the gate/up epilogue (EPI bytes) at the end;
//   two stages of their block scales: fp32 [block of the quad][pair].
// Stages of a quad rather than a turn keep a big item's workgroup at 34 KB, so
// that four fit a CU.
constexpr int qe_cmax(int a, int b) { return a > b ? a : b; }
template <bool GU, int NC, int NT> struct TileLds {
    static constexpr int NB = (GU ? QE_D : QE_FF_EXP) / 32;
    static constexpr int DW = 0, DW_SZ = NB * 4 * 16 * NC * 2;
    static constexpr int EPI = !GU ? 0
                               : NC == 1 ? (2 * 16 * 16 * 4 + 2 * 16 * 4 + 16 * 32 + 2 * 16 * 4) * NT
                                         : 4 * QE_MFMA_MC * 4 + 16 * NT * (64 + 8 + 8);
    static constexpr int ACT = DW + DW_SZ, ACT_SZ = qe_cmax(16 * NT * 128, EPI);
    static constexpr int XS = ACT + 2 * ACT_SZ, XS_SZ = 4 * 16 * NT * 4;
    static constexpr int SIZE = XS + 2 * XS_SZ;
};
template <bool GU> struct ExpertSmem {
    static constexpr int SIZE = qe_cmax(TileLds<GU, 2, 4>::SIZE, qe_cmax(TileLds<GU, 2, 2>::SIZE, TileLds<GU, 2, 1>::SIZE));
    static_assert(TileLds<GU, 1, 2>::SIZE <= SIZE, "the one-matrix gate/up waves fit as well");
    alignas(16) uint8_t raw[SIZE];
    int pair[QE_MFMA_MC];
};

// Wave = NC column groups of 16 weight rows x NT 16-pair tiles (NC MFMAs per
// block and tile; each weight decoded once per item).
// Row groups yb of a workgroup (4 waves):
//   gate/up, NC = 4: h rows 32 (4 yb + wave) + 0..31; groups gate, gate+16, up, up+16;
//   gate/up, NC = 2: h rows 16 (4 yb + wave) + 0..15; groups gate, up -- a 32-block
//            of h spans the wave pair (2w, 2w+1), which meets in LDS for its maximum;
//   gate/up, NC = 1: h rows 32 yb + 16 (wave % 2) + 0..15 of the gate (waves 0, 1) or
//            up (waves 2, 3) matrix -- half the rows of NC = 2 per workgroup, each
//            output's K order unchanged; the up waves hand their dots to the gate
//            waves through LDS;
//   down:    output rows 64 NC yb + 16 NC wave + 16 c + 0..15.
template <bool GU, int NC, int NT>
__device__ __forceinline__ void expert_tile(const GemmTileArgs &a, const int4 it, const int yb, ExpertSmem<GU> &sm) {
    static_assert(NC == 2 || NC == 4 || (GU && NC == 1), "one (gate/up), two or four column groups per wave");
    static_assert(16 * NT <= QE_MFMA_MC, "tiles of the item");
    constexpr int KD = GU ? QE_D : QE_FF_EXP;  // reduction length
    constexpr int NB = KD / 32;                // K blocks
    constexpr int NCH = NB / 8;                // turns (two quads each)
    constexpr uint32_t RB = GU ? QE_GU_ROW_BYTES : QE_DN_ROW_BYTES;
    auto &s_pair = sm.pair;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, n = lane & 15, g = lane >> 4;
    auto row_of = [&](int w, int c, int nn) -> int {
        if constexpr (!GU) return yb * (64 * NC) + w * (16 * NC) + 16 * c + nn;
        else if constexpr (NC == 4) return (c < 2 ? 0 : QE_FF_EXP) + (yb * 4 + w) * 32 + 16 * (c & 1) + nn;
        else if constexpr (NC == 2) return (c == 0 ? 0 : QE_FF_EXP) + (yb * 4 + w) * 16 + nn;
        else return (w < 2 ? 0 : QE_FF_EXP) + (yb * 2 + (w & 1)) * 16 + nn;
    };
    const uint8_t *ebase = a.arena + (size_t)it.x * QE_EXPERT_BYTES + (GU ? 0 : QE_EXPERT_DOWN_OFF);
    // Buffer loads: a range-checked resource per operand (reads past the end
    // return 0), uniform per-turn offsets in SGPRs, per-lane offsets fixed.
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)ebase, (short)0, (int)(GU ? QE_EXPERT_DOWN_OFF : QE_EXPERT_BYTES - QE_EXPERT_DOWN_OFF), 0x00020000);
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc((void *)a.aq, (short)0, a.a_bytes, 0x00020000);
    auto ld128 = [](__amdgpu_buffer_rsrc_t r, uint32_t vo, int so) {
        const qe_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    using LY = TileLds<GU, NC, NT>;
    uint8_t *const lds = sm.raw;

    int rowc[NC];
    uint32_t boff[NC]; // byte offset of block g of the lane's row, per column group
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        rowc[c] = row_of(wv, c, n);
        boff[c] = (uint32_t)rowc[c] * RB + 16 * g;
    }
    // Ring: quad slot qs of turn ch holds blocks 8 ch + 4 qs .. +3; refills wrap
    // to turn (ch + 1) % NCH.
    uint4 rq[2][NC]; // raw codes, per quad slot and column group
    auto load_q = [&](int ch, int qs, uint32_t dep) {
#pragma unroll
        for (int c = 0; c < NC; ++c) rq[qs][c] = ld128(wr, boff[c] + dep, 128 * ch + 64 * qs);
    };

    // Start-up: the loads that depend on the expert only (turn 0 of the code
    // ring, the weight scales) go out before the pairs, which gate the activations.
    load_q(0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_q(0, 1, 0);
    __builtin_amdgcn_sched_barrier(0);
    static_assert(64 * NC <= 256, "one weight row per thread");
    const bool dw_role = tid < 64 * NC; // thread = one weight row of the workgroup: its NB scales
    const int dw_w = tid / (16 * NC), dw_c = (tid >> 4) % NC, dw_n = tid & 15;
    uint4 dwv[NB / 8];
    if (dw_role) {
        const uint4 *sc = (const uint4 *)(ebase + (size_t)row_of(dw_w, dw_c, dw_n) * RB + KD / 2);
#pragma unroll
        for (int i = 0; i < NB / 8; ++i) dwv[i] = sc[i];
    }
    if (tid < QE_MFMA_MC) s_pair[tid] = tid < it.z ? a.pairs[it.y + tid] : -1;
    __syncthreads();

    // Stage roles of this thread, per quad:
    //   activations: pair m = 32 r + tid / 8, chunk q = tid % 8 of the quad, m < 16 NT
    //     (padding pairs load pair 0's row; their scales are 0);
    //   activation scales (tid >= 256 - 16 NT): the quad's four blocks of pair m.
    constexpr int NPASS = (16 * NT + 31) / 32;
    uint32_t act_off[NPASS];
#pragma unroll
    for (int r = 0; r < NPASS; ++r) {
        const int m = 32 * r + (tid >> 3), p = m < 16 * NT ? s_pair[m] : -1;
        act_off[r] = (uint32_t)((p < 0 ? s_pair[0] : p) / a.a_row_div) * KD + 16 * (tid & 7);
    }
    const bool act_role = 32 * (NPASS - 1) + (tid >> 3) < 16 * NT; // the last pass (all passes when NT > 1)
    const int act_st = (tid >> 3) * 128 + (((tid & 7) ^ ((tid >> 4) & 7)) << 4); // + 32 r * 128
    const int xs_m = tid - (256 - 16 * NT);
    const bool xs_role = xs_m >= 0;
    const int xs_p = xs_role ? s_pair[xs_m] : -1;
    const float4 *xs_src = (const float4 *)(a.as + (size_t)((xs_p < 0 ? 0 : xs_p) / a.a_row_div) * NB);
    uint4 sa[NPASS];
    float4 sxs = make_float4(0.f, 0.f, 0.f, 0.f);
    auto stage_load = [&](int qq) {
#pragma unroll
        for (int r = 0; r < NPASS; ++r)
            if (r + 1 < NPASS || act_role) sa[r] = ld128(ar, act_off[r], 128 * qq);
        if (xs_p >= 0) sxs = xs_src[qq];
    };
    auto stage_store = [&](int s) {
        uint8_t *act = lds + LY::ACT + s * LY::ACT_SZ;
#pragma unroll
        for (int r = 0; r < NPASS; ++r)
            if (r + 1 < NPASS || act_role) *(uint4 *)(act + 32 * r * 128 + act_st) = sa[r];
        if (xs_role) {
            float *xs = (float *)(lds + LY::XS + s * LY::XS_SZ) + xs_m;
            xs[0 * 16 * NT] = sxs.x;
            xs[1 * 16 * NT] = sxs.y;
            xs[2 * 16 * NT] = sxs.z;
            xs[3 * 16 * NT] = sxs.w;
        }
    };
    stage_load(0);
    if (dw_role) {
        uint16_t *dwl = (uint16_t *)(lds + LY::DW) + (dw_w * 16 + dw_n) * NC + dw_c;
#pragma unroll
        for (int i = 0; i < NB / 8; ++i) {
            const uint32_t w4[4] = {dwv[i].x, dwv[i].y, dwv[i].z, dwv[i].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) dwl[(8 * i + j) * 64 * NC] = (uint16_t)(w4[j >> 1] >> (16 * (j & 1)));
        }
    }
    stage_store(0);
    __syncthreads();

    float acc[NC][NT][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[c][t][i] = 0.f;

    for (int ch = 0; ch < NCH; ++ch) {
        const int nx = ch + 1 < NCH ? ch + 1 : 0;
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
            // quad qq = 2 ch + qs reads stage qs; the next quad's stage is loaded a quad ahead
            const int qq = 2 * ch + qs;
            const bool more = qq + 1 < 2 * NCH;
            const uint8_t *act = lds + LY::ACT + qs * LY::ACT_SZ;
            const float *xsl = (const float *)(lds + LY::XS + qs * LY::XS_SZ);
            if (more) stage_load(qq + 1);
            __builtin_amdgcn_sched_barrier(0);
            uint32_t cw[NC][4]; // [group][block of the quad]: the lane's code dword
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                // copy out of the ring first: the swaps overwrite their operands, and
                // the ring registers must stay free for the refill
                const uint32_t r4[4] = {rq[qs][c].x, rq[qs][c].y, rq[qs][c].z, rq[qs][c].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) asm volatile("v_mov_b32 %0, %1" : "=v"(cw[c][k]) : "v"(r4[k]));
                transpose_rows4(cw[c]);
            }
            {
                uint32_t dep;
                if constexpr (NC == 4)
                    asm volatile("v_mov_b32 %0, 0" : "=v"(dep)
                                 : "v"(cw[0][0]), "v"(cw[1][0]), "v"(cw[2][0]), "v"(cw[3][0]));
                else if constexpr (NC == 2)
                    asm volatile("v_mov_b32 %0, 0" : "=v"(dep) : "v"(cw[0][0]), "v"(cw[1][0]));
                else
                    asm volatile("v_mov_b32 %0, 0" : "=v"(dep) : "v"(cw[0][0]));
                load_q(nx, qs, dep);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int jp = 0; jp < 2; ++jp) {
                // blocks 2 jp, 2 jp + 1 of the quad: one 16-byte LDS read per tile
                uint4 av2[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    av2[t] = *(const uint4 *)(act + (16 * t + n) * 128 + (((4 * jp + g) ^ (n >> 1)) << 4));
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int j = 2 * jp + jj, s = 4 * qs + j; // block j of the quad, s of the turn
                    long bv[NC];
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        uint32_t lo, hi;
                        nl4_decode_dword<true>(cw[c][j], lo, hi);
                        bv[c] = (long)(((uint64_t)hi << 32) | lo);
                    }
                    // fp16 weight scales, widened once per block: x * dw is then a v_mul_f32,
                    // which issues at twice the rate of the v_fma_mix_f32 the compiler would
                    // otherwise fold the widening into (measured: k_expert_gu -3 % at 512
                    // tokens, -6 % at 8192)
                    typedef _Float16 hNC __attribute__((ext_vector_type(NC)));
                    const hNC dw = *(const hNC *)(lds + LY::DW + (((8 * ch + s) * 4 + wv) * 16 + n) * NC * 2);
                    // dwf = dw, cng = -QE_I2F_MAGIC * dw: exact in fp32 (dw has at most 11
                    // significant bits, 3 dw at most 13, and QE_I2F_MAGIC = 3 * 2^22)
                    float dwf[NC], cng[NC];
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        dwf[c] = (float)dw[c];
                        cng[c] = dwf[c] * -QE_I2F_MAGIC;
                        asm volatile("" : "+v"(dwf[c]), "+v"(cng[c]));
                    }
                    // per tile: NC exact block dots on the matrix cores, each accumulated onto
                    // the bits of QE_I2F_MAGIC, so that read as a float it is QE_I2F_MAGIC + P
                    // exactly (|P| <= 32 * 127 * 127 < 2^22); then fma(D, dw, -QE_I2F_MAGIC dw)
                    // = P * dw with one rounding, and one fma more with the activation scale
                    // (two full-rate fmas per output instead of a conversion, a product and an
                    // fma)
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const uint4 v = av2[t];
                        const long av = jj ? (long)(((uint64_t)v.w << 32) | v.z) : (long)(((uint64_t)v.y << 32) | v.x);
                        typedef int i32x4 __attribute__((ext_vector_type(4)));
                        i32x4 P[NC];
#pragma unroll
                        for (int c = 0; c < NC; ++c) {
                            const i32x4 mag = {QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS};
                            P[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv[c], mag, 0, 0, 0);
                        }
                        const float4 x4 = *(const float4 *)(xsl + j * 16 * NT + 16 * t + 4 * g);
#pragma unroll
                        for (int c = 0; c < NC; ++c) {
                            acc[c][t][0] = fmaf(fmaf(__int_as_float(P[c][0]), dwf[c], cng[c]), x4.x, acc[c][t][0]);
                            acc[c][t][1] = fmaf(fmaf(__int_as_float(P[c][1]), dwf[c], cng[c]), x4.y, acc[c][t][1]);
                            acc[c][t][2] = fmaf(fmaf(__int_as_float(P[c][2]), dwf[c], cng[c]), x4.z, acc[c][t][2]);
                            acc[c][t][3] = fmaf(fmaf(__int_as_float(P[c][3]), dwf[c], cng[c]), x4.w, acc[c][t][3]);
                        }
                    }
                    // scale now: left alone the compiler defers the block's scaling,
                    // keeping every block product of the turn live
#pragma unroll
                    for (int c = 0; c < NC; ++c)
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            asm volatile("" : "+v"(acc[c][t][0]), "+v"(acc[c][t][1]), "+v"(acc[c][t][2]), "+v"(acc[c][t][3]));
                }
            }
            if (more) {
                // the other stage was last read in quad qq - 1, before the previous barrier
                stage_store(qs ^ 1);
                __syncthreads();
            }
        }
    }
    // the last quad (odd) read stage 1: the epilogue works in stage 0

    // lane holds rows 16 t + 4 g + i, column n of each group
    if constexpr (GU && NC == 4) {
        const int jb = yb * 4 + wv; // 32-block of h
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float h0 = silu_mul(acc[0][t][i], acc[2][t][i]);
                const float h1 = silu_mul(acc[1][t][i], acc[3][t][i]);
                float m = fmaxf(fabsf(h0), fabsf(h1));
                m = max16(m);
                float d;
                const float id = quant_scale_inv(m, d);
                const int p = s_pair[16 * t + 4 * g + i];
                if (p >= 0) {
                    int8_t *hrow = a.hq + (size_t)p * QE_FF_EXP + (jb >> 1) * 64 + (n >> 2) * 16 + (jb & 1) * 8 + (n & 3);
                    hrow[0] = quant_one(h0, id);
                    hrow[4] = quant_one(h1, id);
                    if (n == 0) a.hs[(size_t)p * (QE_FF_EXP / 32) + jb] = d;
                }
            }
        }
    } else if constexpr (GU && NC == 1) {
        // 32-block yb of h: rows 16 rs + n, rs = wv % 2, from gate wave rs and up wave
        // 2 + rs.  All of it goes through stage 0, which the last quad did not read.
        uint8_t *fs = sm.raw + LY::ACT;
        float *utile = (float *)fs;                              // [2][16 NT pairs][16] the up dots
        float *amax = utile + 2 * 16 * NT * 16;                  // [2][16 NT] |h| maxima per half
        uint8_t *htile = (uint8_t *)(amax + 2 * 16 * NT);         // [16 NT][32] int8 h, operand order
        float *stile = (float *)(htile + 16 * NT * 32);          // [16 NT] block scales
        float *itile = stile + 16 * NT;                          // [16 NT] their inverses
        static_assert((2 * 16 * 16 * 4 + 2 * 16 * 4 + 16 * 32 + 2 * 16 * 4) * NT <= LY::ACT_SZ,
                      "the epilogue fits the free stage");
        const int rs = wv & 1;
        if (wv >= 2) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) utile[(rs * 16 * NT + 16 * t + 4 * g + i) * 16 + n] = acc[0][t][i];
        }
        __syncthreads();
        float h[NT][4], m[NT][4];
        if (wv < 2) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int mi = 16 * t + 4 * g + i;
                    h[t][i] = silu_mul(acc[0][t][i], utile[(rs * 16 * NT + mi) * 16 + n]);
                    m[t][i] = max16_abs(h[t][i]);
                    if (n == 0) amax[rs * 16 * NT + mi] = m[t][i];
                }
        }
        __syncthreads();
        if (tid < 16 * NT) { // the block's scale and its inverse, once per pair
            float d;
            itile[tid] = quant_scale_inv(fmaxf(amax[tid], amax[16 * NT + tid]), d);
            stile[tid] = d;
        }
        __syncthreads();
        if (wv < 2) {
            // element 16 rs + n of the block: byte (n / 4) * 16 + (yb % 2) * 8 + n % 4 + 4 rs
            // of the pair's 64-byte run (yb / 2) of h (the layout of the NC = 2 path);
            // htile keeps this block's 8-byte groups n / 4 contiguous
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int mi = 16 * t + 4 * g + i;
                    htile[mi * 32 + (n >> 2) * 8 + (n & 3) + 4 * rs] = (uint8_t)quant_one(h[t][i], itile[mi]);
                }
        }
        __syncthreads();
        {   // thread (pair tid / 4, 8-byte group tid % 4)
            const int mi = tid >> 2, q = tid & 3;
            const int p = mi < 16 * NT ? s_pair[mi] : -1;
            if (p >= 0) {
                int8_t *hp = a.hq + (size_t)p * QE_FF_EXP + (yb >> 1) * 64 + 16 * q + 8 * (yb & 1);
                float *sp = a.hs + (size_t)p * (QE_FF_EXP / 32) + yb;
                if (a.item_done) { // fused launch: written through for its down workgroups
                    st_sc1(hp, *(const uint2 *)(htile + mi * 32 + 8 * q));
                    if (q == 0) st_sc1(sp, stile[mi]);
                } else {
                    *(uint2 *)hp = *(const uint2 *)(htile + mi * 32 + 8 * q);
                    if (q == 0) *sp = stile[mi];
                }
            }
        }
    } else if constexpr (GU) {
        // h rows 16 (4 yb + wv) + n: half (wv & 1) of 32-block jb
        const int jb = yb * 2 + (wv >> 1), half = wv & 1;
        // each wave's |h| maximum per pair, in the activation stage the last turn
        // did not read (stage 0: its last reader passed the barrier that ended quad 2 NCH - 2)
        float(*amax)[QE_MFMA_MC] = (float(*)[QE_MFMA_MC])(sm.raw + LY::ACT);
        static_assert(4 * QE_MFMA_MC * 4 <= LY::ACT_SZ, "maxima fit one stage");
        float h[NT][4], m[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[t][i] = silu_mul(acc[0][t][i], acc[1][t][i]);
                m[t][i] = max16_abs(h[t][i]);
                if (n == 0) amax[wv][16 * t + 4 * g + i] = m[t][i];
            }
        __syncthreads();
        // The workgroup's h of a pair is the 64 contiguous bytes [64 yb, 64 yb + 64) of its
        // row in the operand layout (blocks 2 yb, 2 yb + 1), and its two block scales are
        // adjacent: both are assembled in LDS (after the maxima, in the same free stage)
        // and stored 16 bytes per thread, instead of one byte per lane and value.
        uint8_t *htile = sm.raw + LY::ACT + 4 * QE_MFMA_MC * 4; // [16 NT][64]
        float *stile = (float *)(htile + 16 * NT * 64);                                  // [16 NT][2]
        float *itile = stile + 16 * NT * 2;                                              // [2][16 NT] inverses
        static_assert(4 * QE_MFMA_MC * 4 + 16 * NT * (64 + 8 + 8) <= LY::ACT_SZ, "h tile fits the free stage");
        if (tid < 2 * 16 * NT) { // block (jb % 2 = wave pair) scale and its inverse, once per pair
            const int pr = tid / (16 * NT), mi = tid % (16 * NT);
            float d;
            itile[tid] = quant_scale_inv(fmaxf(amax[2 * pr][mi], amax[2 * pr + 1][mi]), d);
            stile[mi * 2 + pr] = d;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 id4 = *(const float4 *)(itile + (wv >> 1) * 16 * NT + 16 * t + 4 * g);
            const float id[4] = {id4.x, id4.y, id4.z, id4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mi = 16 * t + 4 * g + i;
                htile[mi * 64 + (n >> 2) * 16 + (jb & 1) * 8 + (n & 3) + 4 * half] = (uint8_t)quant_one(h[t][i], id[i]);
            }
        }
        __syncthreads();
        {   // thread (pair tid / 4, 16-byte part tid % 4)
            const int mi = tid >> 2, q = tid & 3;
            const int p = mi < 16 * NT ? s_pair[mi] : -1;
            if (p >= 0) {
                int8_t *hp = a.hq + (size_t)p * QE_FF_EXP + (jb >> 1) * 64 + 16 * q;
                float *sp = a.hs + (size_t)p * (QE_FF_EXP / 32) + 2 * (jb >> 1);
                if (a.item_done) { // fused launch: written through for its down workgroups
                    st_sc1(hp, *(const uint4 *)(htile + mi * 64 + 16 * q));
                    if (q == 0) st_sc1(sp, *(const uint2 *)(stile + mi * 2));
                } else {
                    *(uint4 *)hp = *(const uint4 *)(htile + mi * 64 + 16 * q);
                    if (q == 0) *(float2 *)sp = *(const float2 *)(stile + mi * 2);
                }
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = s_pair[16 * t + 4 * g + i];
                if (p < 0) continue;
                const float w = a.wts[p];
                float *yrow = a.yp + (size_t)p * QE_D;
#pragma unroll
                for (int c = 0; c < NC; ++c) yrow[rowc[c]] = w * acc[c][t][i];
            }
        }
    }
}

// Gate/up: big items (33..64 pairs, the first n_items[1]) run NT = 4, NC = 2
// on 8 row groups of 64 h rows; the small ones after them NT = 2 or 1 on
// NC = 1, 16 row groups of 32 h rows: twice the workgroups of half the life
// (these items run last, after the big ones, and their workgroups had made the
// launch's tail).  Workgroup b runs on XCD x = b % 8 (round-robin dispatch) and
// takes the (b / 8)-th row group of that XCD's items x, x + 8, ..., the big
// ones' first: all row groups of an item run on one XCD, so its activations
// come from HBM once and from that XCD's L2 after.  (The odd row groups of a
// big item as empty workgroups instead, interleaved with its real ones, left
// half the CUs without work: the dispatcher deals an XCD's workgroups to its
// CUs in turn.)
template <bool GU> constexpr int expert_rg() { return GU ? QE_FF_EXP / 32 : QE_D / 128; }
template <bool GU> QE_DEV void expert_unit(const GemmTileArgs &a, int b, ExpertSmem<GU> &sm) {
    static_assert(GU, "the down items run dn_unit");
    const int x = b & 7, k = b >> 3, nbig = a.n_items[1];
    const int nbx = nbig > x ? (nbig - x + 7) >> 3 : 0; // big items on this XCD
    const bool big = k < 8 * nbx;
    const int k2 = k - 8 * nbx;
    const int item = x + 8 * (big ? k >> 3 : nbx + (k2 >> 4)), yb = big ? k & 7 : k2 & 15;
    if (item >= a.n_items[0]) return;
    const int4 it = a.items[item];
    static_assert(QE_MFMA_MC == 64, "items of up to four 16-row tiles");
    if (big)
        expert_tile<GU, 2, 4>(a, it, yb, sm);
    else if (it.z > 16)
        expert_tile<GU, 1, 2>(a, it, yb, sm);
    else
        expert_tile<GU, 1, 1>(a, it, yb, sm);
    if (a.item_done) {
        // fused launch: every thread's h stores (sc1, written through) are acknowledged
        // before the item's count of finished gate/up workgroups goes up
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(a.item_done + item, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
// Workgroups over the items of np pairs: an upper bound of the item count
// (items of more than QE_MFMA_MC / 2 pairs, plus at most one smaller item per
// expert) rounded up to whole groups of 8 items, times the row groups.
template <bool GU> constexpr int expert_max_wg(int np) {
    return expert_rg<GU>() * (((np / (QE_MFMA_MC / 2 + 1) + 1 + QE_N_EXPERT) + 7) & ~7);
}
__global__ __launch_bounds__(256, 4) void k_expert_gu(GemmTileArgs a) {
    __shared__ ExpertSmem<true> sm;
    expert_unit<true>(a, blockIdx.x, sm);
}


// ===========================================================================
// Shared expert (Q8 weights, fp32 activations; engine/qe.cpp:2469, :1656,
// :1960-1963) as fp16 MFMA GEMMs.  The activations arrive split into fp16
// hi + lo halves in the interleaved layout of store_hilo16 (k_normq writes xn
// that way, the gate/up epilogue writes h); Q8 values are exact in fp16, so two
// MFMA chains (hi, lo) give each 32-block dot within ~2^-22 of fp32, and the
// block's Q8 scale is one fma per output.
//
// v_mfma_f32_32x32x16_f16: lane l supplies 8 k of row (A) / column (B) l % 32
// and receives D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32], i = 0..15.  Within a
// 32-block, lane (., kh = l / 32) feeds elements 16 kh + 8 s + 0..7 at step
// s = 0, 1 on both operands -- a permutation of the block's k, so the same dot.
// The activations are stored in exactly that order (qe_hl_off), so each of a
// lane's four A chunks per block is one 1 KB-contiguous dwordx4 load, and its
// B operand is one 16-byte run of a Q8 row.
//   gate/up: workgroup = 32 tokens x (gate rows j0..j0+31, up rows j0..j0+31),
//            the four waves split K in quarters, partial sums meet in LDS,
//            h = silu(g) * u is written as hi|lo halves (below 2048 tokens;
//            from there shgu_tile64).
//   down:    workgroup = 64 tokens x 128 output rows, LDS-staged (shdn_tile64).
// Rows T..T+31 of the last tile exist in the buffers (sized for whole tiles) and
// are never stored; each output row depends on its own A row only.
// ===========================================================================
typedef float qe_float16v __attribute__((ext_vector_type(16)));
#define SH_GU_KB 16 /* 32-blocks per wave in gate/up: 2048 / 32 / 4 */

QE_DEV qe_u32x4 sh_ld(__amdgpu_buffer_rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }

// one 32-block: acc += dw * (A_hi + A_lo) . B, A = a[0..3] (hi 0..7, hi 8..15, lo 0..7, lo 8..15)
QE_DEV void sh_block(const qe_u32x4 a[4], qe_u32x4 w, float dw, qe_float16v &acc) {
    // dw widened here, once: folded into each fma it becomes a half-rate v_fma_mix_f32
    asm volatile("" : "+v"(dw));
    const qe_half8 b0 = i8x8_to_half8(w.x, w.y), b1 = i8x8_to_half8(w.z, w.w);
    qe_float16v p = {};
    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qe_half8, a[0]), b0, p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qe_half8, a[2]), b0, p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qe_half8, a[1]), b1, p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(qe_half8, a[3]), b1, p, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = fmaf(dw, p[i], acc[i]);
    // scale now: left alone the compiler defers every block's scaling to the end,
    // keeping all the block products live
    asm volatile("" : "+v"(acc));
}
QE_DEV float half_of(const qe_u32x4 s[2], int b) { // fp16 scale b of 16 packed in two dwordx4
    const uint32_t w = s[b >> 3][(b >> 1) & 3];
    return f16_bits_to_f32((uint16_t)((b & 1) ? w >> 16 : w & 0xffffu));
}

// Router logits 0..255 in the canonical fp32 order, tiled:
// C[m][n] = sum_k xn[m][k] W[n][k].  Canonical order: per 32-wide k chunk an fma
// chain from 0, chunk sums merged by the pairwise tree (chunks (c, c+1), then
// pairs of pairs, ...).  The K range is split eight ways along that tree: split
// z computes the 8-chunk subtree [8z, 8z+8) exactly, and k_topk forms the top
// three levels ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)) -- bit-identical
// to the unsplit order.  Row 256 (the shared-expert gate) is one canonical wave
// dot per token in k_normq.  Tile 64 tokens x 64 rows, 256 threads, 4 x 4 outputs
// per thread; chunks are double-buffered in LDS, k-major, the next one loaded
// into registers while the current one is multiplied.  The transposing stores
// XOR the column with the k group ((k / 8) % 4 * 16), so the four k groups a
// wave stores land in different banks; the reads undo it (float4 runs stay
// aligned).
struct RouterSmem {
    float As[2][32][64];
    float Bs[2][32][64];
};
QE_DEV void router_tile(const float *xn, int T, const float *W, float *part, int n_tile, int m_tile, int z,
                        RouterSmem &sm) {
    constexpr int NCH = 64 / RT_SPLIT; // chunks per split
    auto &As = sm.As;
    auto &Bs = sm.Bs;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = m_tile * 64, n0 = n_tile * 64;
    const int lr = tid >> 2, lk = (tid & 3) * 8; // loader: row lr of the tile, 8 k values
    const bool a_ok = m0 + lr < T;
    const float *ap = xn + (size_t)(a_ok ? m0 + lr : 0) * QE_D + z * NCH * 32 + lk;
    const float *bp = W + (size_t)(n0 + lr) * QE_D + z * NCH * 32 + lk;
    float4 pa[2], pb[2];
    auto fetch = [&](int cl) {
        const float4 *a4 = (const float4 *)(ap + cl * 32), *b4 = (const float4 *)(bp + cl * 32);
        pa[0] = a_ok ? a4[0] : make_float4(0.f, 0.f, 0.f, 0.f);
        pa[1] = a_ok ? a4[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        pb[0] = b4[0];
        pb[1] = b4[1];
    };
    auto stage = [&](int buf) {
        const float va[8] = {pa[0].x, pa[0].y, pa[0].z, pa[0].w, pa[1].x, pa[1].y, pa[1].z, pa[1].w};
        const float vb[8] = {pb[0].x, pb[0].y, pb[0].z, pb[0].w, pb[1].x, pb[1].y, pb[1].z, pb[1].w};
        const int col = lr ^ ((lk >> 3) << 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            As[buf][lk + i][col] = va[i];
            Bs[buf][lk + i][col] = vb[i];
        }
    };
    fetch(0);
    stage(0);
    __syncthreads();
    float st[4][4][4];
#pragma unroll 1
    for (int cl = 0; cl < NCH; ++cl) {
        const int buf = cl & 1;
        if (cl + 1 < NCH) fetch(cl + 1);
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
#pragma unroll
        for (int kk = 0; kk < 32; ++kk) {
            const int sw = ((kk >> 3) & 3) << 4;
            const float4 av = *(const float4 *)&As[buf][kk][(ty * 4) ^ sw];
            const float4 bv = *(const float4 *)&Bs[buf][kk][(tx * 4) ^ sw];
            const float ar[4] = {av.x, av.y, av.z, av.w}, br[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(ar[i], br[j], acc[i][j]);
        }
        bool carry = true; // pairwise-tree merge of chunk cl
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            if (carry) {
                if (cl & (1 << l)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[i][j] = st[l][i][j] + acc[i][j];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) st[l][i][j] = acc[i][j];
                    carry = false;
                }
            }
        }
        if (cl + 1 < NCH) stage(buf ^ 1);
        __syncthreads();
    }
    constexpr int TOP = NCH == 8 ? 3 : NCH == 16 ? 4 : 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= T) continue;
        *(float4 *)&part[((size_t)z * T + m) * QE_N_EXPERT + n0 + tx * 4] =
            make_float4(st[TOP][i][0], st[TOP][i][1], st[TOP][i][2], st[TOP][i][3]);
    }
}

struct ShguSmem {
    float red[4][2][16][64];
};
QE_DEV void shgu_tile(const _Float16 *xhl, int T, const uint8_t *W, _Float16 *hhl, int m_tile, int j_tile, ShguSmem &sm) {
    constexpr uint32_t RB = QE_SH_GU_ROW_BYTES;
    auto &red = sm.red;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 31, kh = lane >> 5;
    const int m0 = m_tile * 32, j0 = j_tile * 32, kb0 = wv * SH_GU_KB;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)xhl, (short)0, ((T + 31) & ~31) * QE_D * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)W, (short)0, (int)QE_SH_GU_BYTES, 0x00020000);
    const uint32_t a_off = (uint32_t)(m_tile * (QE_D / 32) + kb0) * 4096 + lane * 16;
    const uint32_t g_off = (uint32_t)(j0 + c) * RB, u_off = g_off + QE_FF_SH * RB;
    qe_u32x4 sg[2], su[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        sg[i] = sh_ld(rw, g_off + QE_D + 2 * kb0 + 16 * i);
        su[i] = sh_ld(rw, u_off + QE_D + 2 * kb0 + 16 * i);
    }
    qe_float16v ag = {}, au = {};
    constexpr int DEPTH = 3;
    qe_u32x4 ra_[DEPTH][4], rg[DEPTH], ru[DEPTH];
    auto load = [&](int b) {
        const int s = b % DEPTH;
#pragma unroll
        for (int q = 0; q < 4; ++q) ra_[s][q] = sh_ld(ra, a_off + 4096 * b + 1024 * q);
        rg[s] = sh_ld(rw, g_off + 32 * (kb0 + b) + 16 * kh);
        ru[s] = sh_ld(rw, u_off + 32 * (kb0 + b) + 16 * kh);
    };
#pragma unroll
    for (int b = 0; b < DEPTH; ++b) load(b);
#pragma unroll
    for (int b = 0; b < SH_GU_KB; ++b) {
        const int s = b % DEPTH;
        const qe_u32x4 a[4] = {ra_[s][0], ra_[s][1], ra_[s][2], ra_[s][3]};
        const qe_u32x4 wg = rg[s], wu = ru[s];
        if (b + DEPTH < SH_GU_KB) load(b + DEPTH);
        sh_block(a, wg, half_of(sg, b), ag);
        sh_block(a, wu, half_of(su, b), au);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        red[wv][0][i][lane] = ag[i];
        red[wv][1][i][lane] = au[i];
    }
    __syncthreads();
    // thread: lane L of the accumulators, i = 4 (tid / 64) .. +3 -> 4 (token, j) outputs
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = 4 * wv + q;
        const float g = (red[0][0][i][lane] + red[1][0][i][lane]) + (red[2][0][i][lane] + red[3][0][i][lane]);
        const float u = (red[0][1][i][lane] + red[1][1][i][lane]) + (red[2][1][i][lane] + red[3][1][i][lane]);
        const int m = m0 + 8 * (i >> 2) + 4 * kh + (i & 3), j = j0 + c;
        if (m < T) {
            const float h = silu_mul(g, u);
            const _Float16 hi = (_Float16)h, lo = (_Float16)(h - (float)hi);
            uint8_t *dst = (uint8_t *)hhl + qe_hl_off(QE_FF_SH, m, j);
            *(_Float16 *)dst = hi;
            *(_Float16 *)(dst + QE_HL_LO) = lo;
        }
    }
}


// Router split tiles and shared gate/up tiles in one launch, so the fp32 VALU
// router and the matrix-core shared GEMM share the CUs instead of running back
// to back.  Workgroup b runs on XCD b % 8 (the dispatcher deals workgroups
// round robin over the 8 XCDs, each with its own L2), and the tasks are dealt
// so that every XCD gets both kinds, interleaved, and the tiles that share an
// operand run on one XCD back to back: the 4 router column tiles of one
// (token tile, K split) and the 16 shared gate/up row tiles of one token tile.
constexpr int RS_NT = QE_N_EXPERT / 64, RS_JT = QE_FF_SH / 32;
QE_DEV int rs_router_per_xcd(int T) { return RS_NT * ((T + 63) / 64) * RT_SPLIT / 8; }
QE_DEV int rs_shgu_per_xcd(int T, int x) { return RS_JT * (((T + 31) / 32 - x + 7) / 8); }
__global__ __launch_bounds__(256) void k_router_shgu(const float *xn, const _Float16 *xhl, int T, const float *Wr,
                                                     const uint8_t *Wg, float *part, _Float16 *hhl) {
    __shared__ union {
        RouterSmem r;
        ShguSmem s;
    } sm;
    static_assert(RT_SPLIT % 8 == 0, "router groups divide evenly over the XCDs");
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int mt64 = (T + 63) / 64;
    const int nr = rs_router_per_xcd(T), ns = rs_shgu_per_xcd(T, x), both = 2 * (nr < ns ? nr : ns);
    bool router;
    int idx;
    if (k < both) {
        router = (k & 1) == 0;
        idx = k >> 1;
    } else {
        router = nr > ns;
        idx = k - both + (both >> 1);
    }
    if (router) {
        if (idx >= nr) return;
        const int g = 8 * (idx / RS_NT) + x; // (token tile, K split) group
        router_tile(xn, T, Wr, part, idx % RS_NT, g % mt64, g / mt64, sm.r);
    } else {
        if (idx >= ns) return;
        shgu_tile(xhl, T, Wg, hhl, 8 * (idx / RS_JT) + x, idx % RS_JT, sm.s);
    }
}

// From QE_RS_SPLIT_T tokens on, the two kinds run as two launches instead: the
// shared gate/up tiles hold 128 AGPRs, which caps the fused kernel at 2 waves
// per SIMD, while the router tiles alone (128 VGPRs) run 4.  One wave issues a
// VALU instruction only every ~5 cycles, so the fp32 router needs the waves
// (8192 tokens: fused 266 us; router 117 + shared 131 us).  At 512 tokens the
// fused launch is 9 us faster (20 against 17 + 12).
#define QE_RS_SPLIT_T 2048
__global__ __launch_bounds__(256) void k_router(const float *xn, int T, const float *Wr, float *part) {
    __shared__ RouterSmem sm;
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3, mt64 = (T + 63) / 64;
    const int g = 8 * (k / RS_NT) + x;
    router_tile(xn, T, Wr, part, k % RS_NT, g % mt64, g / mt64, sm);
}
// Shared gate/up for large T: workgroup = 64 tokens (two 32-token tiles) x 64
// gate rows + the same 64 up rows; wave w takes token tile w & 1 and rows
// 32 (w >> 1) + 0..31 of both, over the full K, so no partial sums meet.  Each
// 32-block of K, the workgroup stages the 8 KB of activations and 4 KB of Q8
// rows in LDS once (double-buffered, one barrier per block) and every wave reads
// its operands from there: each fetched byte feeds two waves' MFMAs instead of
// one.  The Q8 block scales of the 128 rows sit in LDS for the whole K, block-
// major, so the 32 rows a wave reads for one block are consecutive.
struct Shgu64Smem {
    alignas(16) uint8_t a[2][2][4096]; // [stage][token tile][32-block of hi|lo halves, qe_hl_off order]
    alignas(16) uint8_t w[2][128][32]; // [stage][row: gate 0..63, up 64..127][32 int8]
    _Float16 sc[QE_D / 32][128];       // [block][row]
};
QE_DEV void shgu_tile64(const _Float16 *xhl, int T, const uint8_t *W, _Float16 *hhl, int mp, int jg, Shgu64Smem &sm) {
    constexpr uint32_t RB = QE_SH_GU_ROW_BYTES;
    constexpr int NB = QE_D / 32;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 31, kh = lane >> 5;
    const int mt32 = (T + 31) / 32, j0 = jg * 64;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)xhl, (short)0, mt32 * 32 * QE_D * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)W, (short)0, (int)QE_SH_GU_BYTES, 0x00020000);
    auto row_off = [&](int r) -> uint32_t { return (uint32_t)((r < 64 ? 0 : QE_FF_SH - 64) + j0 + r) * RB; };
    // block scales of the 128 rows: thread (row tid / 2, half tid & 1) brings 32 of them
    {
        const int r = tid >> 1, h = tid & 1;
        qe_u32x4 s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = sh_ld(rw, row_off(r) + QE_D + 64 * h + 16 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t v = s[i][e >> 1];
                sm.sc[32 * h + 8 * i + e][r] = __builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? v >> 16 : v & 0xffffu));
            }
    }
    // staging roles: chunks tid, tid + 256 (activations of token tile 0, 1), tid + 512 (rows)
    uint32_t a_src[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int mt = 2 * mp + s < mt32 ? 2 * mp + s : mt32 - 1; // a tile past T reads the last one; never stored
        a_src[s] = (uint32_t)mt * NB * 4096 + 16 * tid;
    }
    const int wr = tid >> 1, wh = tid & 1;
    const uint32_t w_src = row_off(wr) + 16 * wh;
    qe_u32x4 st[3];
    auto fetch = [&](int b) {
        st[0] = sh_ld(ra, a_src[0] + 4096 * b);
        st[1] = sh_ld(ra, a_src[1] + 4096 * b);
        st[2] = sh_ld(rw, w_src + 32 * b);
    };
    auto put = [&](int s) {
        *(qe_u32x4 *)&sm.a[s][0][16 * tid] = st[0];
        *(qe_u32x4 *)&sm.a[s][1][16 * tid] = st[1];
        *(qe_u32x4 *)&sm.w[s][wr][16 * wh] = st[2];
    };
    fetch(0);
    put(0);
    __syncthreads();
    const int ms = wv & 1, rg = 32 * (wv >> 1) + c, ru = 64 + rg;
    qe_float16v ag = {}, au = {};
#pragma unroll 2
    for (int b = 0; b < NB; ++b) {
        const int s = b & 1;
        if (b + 1 < NB) fetch(b + 1);
        qe_u32x4 a[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = *(const qe_u32x4 *)&sm.a[s][ms][1024 * q + 16 * lane];
        const qe_u32x4 wg = *(const qe_u32x4 *)&sm.w[s][rg][16 * kh], wu = *(const qe_u32x4 *)&sm.w[s][ru][16 * kh];
        sh_block(a, wg, (float)sm.sc[b][rg], ag);
        sh_block(a, wu, (float)sm.sc[b][ru], au);
        if (b + 1 < NB) put(s ^ 1); // stage s ^ 1 was last read in block b - 1, before the barrier
        __syncthreads();
    }
    const int m0 = 64 * mp + 32 * ms, j = j0 + 32 * (wv >> 1) + c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + 8 * (i >> 2) + 4 * kh + (i & 3);
        if (m < T) {
            const float h = silu_mul(ag[i], au[i]);
            const _Float16 hi = (_Float16)h, lo = (_Float16)(h - (float)hi);
            uint8_t *dst = (uint8_t *)hhl + qe_hl_off(QE_FF_SH, m, j);
            *(_Float16 *)dst = hi;
            *(_Float16 *)(dst + QE_HL_LO) = lo;
        }
    }
}
// workgroup b on XCD b % 8: the 8 row groups of one 64-token pair back to back there
__global__ __launch_bounds__(256) void k_shgu(const _Float16 *xhl, int T, const uint8_t *Wg, _Float16 *hhl) {
    __shared__ Shgu64Smem sm;
    const int x = blockIdx.x & 7, k = blockIdx.x >> 3, mp = 8 * (k / 8) + x;
    if (mp >= (T + 63) / 64) return;
    shgu_tile64(xhl, T, Wg, hhl, mp, k % 8, sm);
}

// Shared down, 64 tokens x 128 output rows per workgroup: wave w takes token
// tile w & 1 and rows 64 (w >> 1) + 0..63 (two 32-row MFMA tiles) over the full
// K = 512.  Per 32-block the workgroup stages 8 KB of h halves and 4 KB of Q8
// rows in LDS once (double-buffered), so every fetched byte feeds two waves; the
// 128 rows' block scales sit in LDS block-major for the whole K.  It runs in the
// routed down kernel's LDS (28 KB of its 40).
struct Shdn64Lds {
    alignas(16) uint8_t a[2][2][4096];   // [stage][token tile][32-block of hi|lo halves]
    alignas(16) uint8_t w[2][128][32];   // [stage][row][32 int8]
    _Float16 sc[QE_FF_SH / 32][128];     // [block][row]
};
QE_DEV void shdn_tile64(const _Float16 *hhl, int T, const uint8_t *W, float *out, int mp, int n_tile, uint8_t *lds) {
    constexpr uint32_t RB = QE_SH_DN_ROW_BYTES;
    constexpr int NB = QE_FF_SH / 32;
    Shdn64Lds &sm = *(Shdn64Lds *)lds;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, c = lane & 31, kh = lane >> 5;
    const int mt32 = (T + 31) / 32, n0 = n_tile * 128;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)hhl, (short)0, mt32 * 32 * QE_FF_SH * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)W, (short)0, (int)QE_SH_DN_BYTES, 0x00020000);
    {   // block scales: thread (row tid / 2, half tid & 1) brings 8 of the row's 16
        const int r = tid >> 1, h = tid & 1;
        const qe_u32x4 s = sh_ld(rw, (uint32_t)(n0 + r) * RB + QE_FF_SH + 16 * h);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t v = s[e >> 1];
            sm.sc[8 * h + e][r] = __builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? v >> 16 : v & 0xffffu));
        }
    }
    uint32_t a_src[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int mt = 2 * mp + s < mt32 ? 2 * mp + s : mt32 - 1; // a tile past T reads the last one; never stored
        a_src[s] = (uint32_t)mt * NB * 4096 + 16 * tid;
    }
    const int wr = tid >> 1, wh = tid & 1;
    const uint32_t w_src = (uint32_t)(n0 + wr) * RB + 16 * wh;
    qe_u32x4 st[3];
    auto fetch = [&](int b) {
        st[0] = sh_ld(ra, a_src[0] + 4096 * b);
        st[1] = sh_ld(ra, a_src[1] + 4096 * b);
        st[2] = sh_ld(rw, w_src + 32 * b);
    };
    auto put = [&](int s) {
        *(qe_u32x4 *)&sm.a[s][0][16 * tid] = st[0];
        *(qe_u32x4 *)&sm.a[s][1][16 * tid] = st[1];
        *(qe_u32x4 *)&sm.w[s][wr][16 * wh] = st[2];
    };
    fetch(0);
    put(0);
    __syncthreads();
    const int ms = wv & 1, r0 = 64 * (wv >> 1) + c, r1 = r0 + 32;
    qe_float16v acc0 = {}, acc1 = {};
#pragma unroll 2
    for (int b = 0; b < NB; ++b) {
        const int s = b & 1;
        if (b + 1 < NB) fetch(b + 1);
        qe_u32x4 av[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) av[q] = *(const qe_u32x4 *)&sm.a[s][ms][1024 * q + 16 * lane];
        const qe_u32x4 w0 = *(const qe_u32x4 *)&sm.w[s][r0][16 * kh], w1 = *(const qe_u32x4 *)&sm.w[s][r1][16 * kh];
        sh_block(av, w0, (float)sm.sc[b][r0], acc0);
        sh_block(av, w1, (float)sm.sc[b][r1], acc1);
        if (b + 1 < NB) put(s ^ 1); // stage s ^ 1 was last read in block b - 1, before the barrier
        __syncthreads();
    }
    const int m0 = 64 * mp + 32 * ms;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + 8 * (i >> 2) + 4 * kh + (i & 3);
        if (m < T) {
            out[(size_t)m * QE_D + n0 + r0] = acc0[i];
            out[(size_t)m * QE_D + n0 + r1] = acc1[i];
        }
    }
}

// Routed down of one item over nrg row groups of 128 output rows.  K is only
// 16 blocks, so the item's whole h (up to 64 pairs x 512 int8 in the operand
// layout, 32 KB) and its block scales are staged in LDS once, and each wave then
// streams its 32 rows (two 16-row column groups) of every row group through the
// code ring with no further barrier: one staging of the activations and one
// start-up for 128 nrg rows, where a workgroup per row group paid both per 128.
// The code ring holds two quads (4 blocks each) of both column groups, and
// with them the quad's four weight scales; quad qi is blocks 4 (qi % 4) .. + 3
// of row group rg0 + qi / 4, refilled two quads ahead (the last refills read
// the last quad again).  Arithmetic as expert_tile: exact int8 block dots
// accumulated onto QE_I2F_MAGIC, two fmas per output and block.
struct DnSmem {
    alignas(16) uint8_t act[QE_MFMA_MC * QE_FF_EXP]; // [pair][512 B], 16-byte chunk q of pair m at q ^ (m % 16)
    float xs[QE_FF_EXP / 32][QE_MFMA_MC];           // [block][pair] activation block scales
    float w[QE_MFMA_MC];                            // pair weights
    int pair[QE_MFMA_MC];
};
template <int NT, bool FUSED>
__device__ __forceinline__ void dn_tile(const GemmTileArgs &a, const int4 it, const int rg0, const int nrg, DnSmem &sm) {
    constexpr int NC = 2;
    constexpr uint32_t RB = QE_DN_ROW_BYTES;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, n = lane & 15, g = lane >> 4;
    const uint8_t *dbase = a.arena + (size_t)it.x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)dbase, (short)0, (int)(QE_EXPERT_BYTES - QE_EXPERT_DOWN_OFF), 0x00020000);
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc((void *)a.aq, (short)0, a.a_bytes, 0x00020000);
    const int nq = 4 * nrg;
    uint4 rq[2][NC]; // codes: lane (n, g) holds block 4 Q + g of its row
    uint2 rs[2][NC]; // the quad's four fp16 weight scales of the lane's row
    auto load_quad = [&](int qi, int slot, uint32_t dep) {
        qi = qi < nq ? qi : nq - 1;
        const int Q = qi & 3;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint32_t row = (uint32_t)(128 * (rg0 + (qi >> 2)) + 32 * wv + 16 * c + n) * RB + dep;
            const qe_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, row + 16 * g, 64 * Q, 0);
            rq[slot][c] = make_uint4(v.x, v.y, v.z, v.w);
            const qe_u32x2 sv = __builtin_amdgcn_raw_buffer_load_b64(wr, row + QE_FF_EXP / 2, 8 * Q, 0);
            rs[slot][c] = make_uint2(sv.x, sv.y);
        }
    };
    load_quad(0, 0, 0);
    load_quad(1, 1, 0);
    if (tid < QE_MFMA_MC) {
        const int p = tid < it.z ? a.pairs[it.y + tid] : -1;
        sm.pair[tid] = p;
        sm.w[tid] = p >= 0 ? a.wts[p] : 0.f;
    }
    __syncthreads();
    {   // activations: thread (pair (tid / 16) + 16 r, chunks (tid % 16) + 16 h); scales: (pair tid / 4, blocks 4 (tid % 4) + 0..3)
        uint4 v[NT][2];
#pragma unroll
        for (int r = 0; r < NT; ++r) {
            const int m = (tid >> 4) + 16 * r, pm = sm.pair[m];
            const uint32_t src = (uint32_t)(pm < 0 ? sm.pair[0] : pm) * QE_FF_EXP + 16 * (tid & 15);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // fused launch: h of this launch's gate/up workgroups, from the coherence point (sc1)
                const qe_u32x4 t4 = __builtin_amdgcn_raw_buffer_load_b128(ar, src, 256 * h, FUSED ? 16 : 0);
                v[r][h] = make_uint4(t4.x, t4.y, t4.z, t4.w);
            }
        }
        float4 sc = make_float4(0.f, 0.f, 0.f, 0.f);
        const bool sc_role = tid < 64 * NT;
        const int sm_m = tid >> 2;
        if (sc_role) {
            const int pm = sm.pair[sm_m];
            if (pm >= 0) {
                const float4 *sp = (const float4 *)(a.as + (size_t)pm * (QE_FF_EXP / 32)) + (tid & 3);
                sc = FUSED ? ld_sc1_f4(sp) : *sp;
            }
        }
#pragma unroll
        for (int r = 0; r < NT; ++r) {
            const int m = (tid >> 4) + 16 * r;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                *(uint4 *)(sm.act + m * QE_FF_EXP + ((((tid & 15) + 16 * h) ^ (m & 15)) << 4)) = v[r][h];
        }
        if (sc_role) {
            const int b0 = 4 * (tid & 3);
            sm.xs[b0][sm_m] = sc.x;
            sm.xs[b0 + 1][sm_m] = sc.y;
            sm.xs[b0 + 2][sm_m] = sc.z;
            sm.xs[b0 + 3][sm_m] = sc.w;
        }
    }
    __syncthreads();

    float acc[NC][NT][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[c][t][i] = 0.f;
    auto quad = [&](int qi, int slot) {
        uint32_t cw[NC][4], sw[NC][2];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            // out of the ring first: the swaps overwrite their operands, and the
            // ring registers must stay free for the refill
            const uint32_t r4[4] = {rq[slot][c].x, rq[slot][c].y, rq[slot][c].z, rq[slot][c].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) asm volatile("v_mov_b32 %0, %1" : "=v"(cw[c][k]) : "v"(r4[k]));
            asm volatile("v_mov_b32 %0, %1" : "=v"(sw[c][0]) : "v"(rs[slot][c].x));
            asm volatile("v_mov_b32 %0, %1" : "=v"(sw[c][1]) : "v"(rs[slot][c].y));
            transpose_rows4(cw[c]);
        }
        {
            uint32_t dep;
            asm volatile("v_mov_b32 %0, 0" : "=v"(dep) : "v"(cw[0][0]), "v"(cw[1][0]), "v"(sw[0][0]), "v"(sw[1][0]));
            load_quad(qi + 2, slot, dep);
            __builtin_amdgcn_sched_barrier(0);
        }
        const int Q = qi & 3;
        uint4 av2[NT]; // 16 bytes per tile: the lane's activations of blocks b, b + 1 (b even)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int b = 4 * Q + k;
            if ((k & 1) == 0) {
                // one 16-byte read per tile and block pair: a quarter wave (16 lanes,
                // one lane group g) covers 16 distinct chunks, i.e. all 64 banks
                const int cho = ((2 * Q + (k >> 1)) * 4 + g) ^ n;
#pragma unroll
                for (int t = 0; t < NT; ++t) av2[t] = *(const uint4 *)(sm.act + (16 * t + n) * QE_FF_EXP + (cho << 4));
            }
            long bv[NC];
            float dwf[NC], cng[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                uint32_t lo, hi;
                nl4_decode_dword<true>(cw[c][k], lo, hi);
                bv[c] = (long)(((uint64_t)hi << 32) | lo);
                const uint32_t hw = sw[c][k >> 1] >> (16 * (k & 1));
                dwf[c] = f16_bits_to_f32((uint16_t)hw);
                cng[c] = dwf[c] * -QE_I2F_MAGIC;
                asm volatile("" : "+v"(dwf[c]), "+v"(cng[c]));
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const long av = (k & 1) ? (long)(((uint64_t)av2[t].w << 32) | av2[t].z) : (long)(((uint64_t)av2[t].y << 32) | av2[t].x);
                typedef int i32x4 __attribute__((ext_vector_type(4)));
                i32x4 P[NC];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const i32x4 mag = {QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS, QE_I2F_MAGIC_BITS};
                    P[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv[c], mag, 0, 0, 0);
                }
                const float4 x4 = *(const float4 *)&sm.xs[b][16 * t + 4 * g];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    acc[c][t][0] = fmaf(fmaf(__int_as_float(P[c][0]), dwf[c], cng[c]), x4.x, acc[c][t][0]);
                    acc[c][t][1] = fmaf(fmaf(__int_as_float(P[c][1]), dwf[c], cng[c]), x4.y, acc[c][t][1]);
                    acc[c][t][2] = fmaf(fmaf(__int_as_float(P[c][2]), dwf[c], cng[c]), x4.z, acc[c][t][2]);
                    acc[c][t][3] = fmaf(fmaf(__int_as_float(P[c][3]), dwf[c], cng[c]), x4.w, acc[c][t][3]);
                }
            }
            // scale now: left alone the compiler defers the block's scaling,
            // keeping every block product live
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    asm volatile("" : "+v"(acc[c][t][0]), "+v"(acc[c][t][1]), "+v"(acc[c][t][2]), "+v"(acc[c][t][3]));
        }
        if (Q == 3) { // the row group is complete: yp[p][row] = w_p * y, accumulators cleared
            // lane n holds rows n (c = 0) and 16 + n (c = 1) of the wave's 32; lanes n and
            // n ^ 1 swap a value, so the even one stores rows n, n + 1 and the odd one rows
            // 15 + n, 16 + n as 8-byte pairs: the 16 lanes of a pair write its 128 bytes
            // as one line instead of two half lines
            // The store address is a wave-uniform base (row group, wave) plus a 32-bit
            // lane offset pm * 8192 + 4 col (pm < 2^19 pairs), one VALU instruction per
            // store where 64-bit address arithmetic took six.
            const int rg = rg0 + (qi >> 2);
            const bool odd = n & 1;
            static_assert(QE_D * 4 == 1 << 13 && QE_LAYER_T_MAX * QE_K_USED <= 1 << 19, "offsets fit 32 bits");
            const char *ybase = (const char *)(a.yp + 128 * rg + 32 * __builtin_amdgcn_readfirstlane(wv));
            const uint32_t col4 = 4u * (odd ? 15 + n : n);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 16 * t + 4 * g + i, pm = sm.pair[m];
                    const float w = sm.w[m];
                    const float y0 = w * acc[0][t][i], y1 = w * acc[1][t][i];
                    const float p0 = dpp_f<QE_DPP_XOR1>(y0), p1 = dpp_f<QE_DPP_XOR1>(y1);
                    if (pm >= 0)
                        *(float2 *)(ybase + (((uint32_t)pm << 13) | col4)) =
                            odd ? make_float2(p1, y1) : make_float2(y0, p0);
#pragma unroll
                    for (int c = 0; c < NC; ++c) acc[c][t][i] = 0.f;
                }
        }
    };
    for (int qi = 0; qi < nq; qi += 2) {
        quad(qi, 0);
        quad(qi + 1, 1);
    }
}

// Down workgroup b: item and row-group block; all row-group blocks of an item
// on one XCD (b % 8), as for gate/up.  Big items run NT = 4, smaller NT = 2, 1.
template <bool FUSED> __device__ __forceinline__ void dn_unit_at(const GemmTileArgs &a, int item, int rgb, DnSmem &sm) {
    const int4 it = a.items[item];
    static_assert(QE_MFMA_MC == 64, "items of up to four 16-row tiles");
    if constexpr (FUSED) {
        // the item's gate/up workgroups (8 row groups of a big item, 16 of a small one)
        // come earlier in the grid, so all have started; a bounded wait all the same
        if (threadIdx.x == 0) {
            const int need = (it.z > QE_MFMA_MC / 2 ? 8 : 16) + a.wait_extra;
            for (int spins = 0;; ++spins) {
                if (__hip_atomic_load(a.item_done + item, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= need) break;
                if (spins + 1 >= a.spin_cap) {
                    __hip_atomic_store(a.err, a.err_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        __syncthreads();
    }
    if (it.z > 32)
        dn_tile<4, FUSED>(a, it, rgb * a.dn_rgw, a.dn_rgw, sm);
    else if (it.z > 16)
        dn_tile<2, FUSED>(a, it, rgb * a.dn_rgw, a.dn_rgw, sm);
    else
        dn_tile<1, FUSED>(a, it, rgb * a.dn_rgw, a.dn_rgw, sm);
}
__device__ __forceinline__ void dn_unit(const GemmTileArgs &a, int b, DnSmem &sm) {
    const int rgb_n = (QE_D / 128) / a.dn_rgw; // row-group blocks per item
    const int k = b >> 3, item = (k / rgb_n) * 8 + (b & 7), rgb = k % rgb_n;
    if (item >= a.n_items[0]) return;
    dn_unit_at<false>(a, item, rgb, sm);
}
// workgroups of the routed down over the items of np pairs (as expert_max_wg)
QE_HD int dn_max_wg(int np, int rgw) { return ((QE_D / 128) / rgw) * (((np / (QE_MFMA_MC / 2 + 1) + 1 + QE_N_EXPERT) + 7) & ~7); }

// Routed down items and shared down tiles in one launch: the routed items
// (item, then row-group block) come first, the shared tiles fill the CUs as the
// routed work drains.
__global__ __launch_bounds__(256, 2) void k_expert_dn(GemmTileArgs a, int nr, const _Float16 *hhl, int T,
                                                      const uint8_t *Wsd, float *sd) {
    __shared__ union {
        DnSmem d;
        Shdn64Lds s;
    } sm;
    const int b = blockIdx.x;
    if (b < nr) {
        dn_unit(a, b, sm.d);
    } else {
        const int s = b - nr;
        // tile s runs on XCD s % 8 (nr is a multiple of 8 below): the 16 column
        // tiles of one 64-token pair back to back there
        const int x = s & 7, k = s >> 3, mp = 8 * (k / (QE_D / 128)) + x;
        if (mp >= (T + 63) / 64) return;
        shdn_tile64(hhl, T, Wsd, sd, mp, k % (QE_D / 128), (uint8_t *)&sm.s);
    }
}

// From QE_FUSE_T_MIN to QE_FUSE_T tokens the routed gate/up, the routed down and
// the shared down run as one launch: the down workgroups alone would leave CUs
// idle, and the gate/up work ends in a tail of small items.  Workgroup b runs on XCD x = b % 8
// and is the (b / 8)-th of that XCD's sequence, laid out from the item counts:
// its items' gate/up workgroups (as k_expert_gu), the shared down tiles of the
// XCD (they wait for nothing), its items' down workgroups (big items first),
// then nothing (the grid is an upper bound).  A down workgroup waits until its
// item's gate/up workgroups have counted themselves done (their h written
// through, sc1, and acknowledged first) and stages h from the coherence point.
// The dispatcher starts an XCD's workgroups in grid order, so every gate/up
// workgroup a down one waits for has started.
#ifndef QE_FUSE_T_MIN
#define QE_FUSE_T_MIN 32
#endif
#ifndef QE_FUSE_T
#define QE_FUSE_T 4096
#endif
__global__ __launch_bounds__(256, 4) void k_expert_gudn(GemmTileArgs gu, GemmTileArgs dn, int nshx,
                                                        const _Float16 *hhl, int T, const uint8_t *Wsd, float *sd) {
    __shared__ union {
        ExpertSmem<true> g;
        DnSmem d;
        Shdn64Lds s;
    } sm;
    const int b = blockIdx.x, x = b & 7, k = b >> 3;
    const int ni = gu.n_items[0], nb = gu.n_items[1];
    const int nix = ni > x ? (ni - x + 7) >> 3 : 0, nbx = nb > x ? (nb - x + 7) >> 3 : 0; // items x, x + 8, ..
    const int gux = 8 * nbx + 16 * (nix - nbx);
    if (k < gux) {
        expert_unit<true>(gu, b, sm.g);
        return;
    }
    int r = k - gux;
    if (r < nshx) { // shared tile s = 8 r + x: the 16 column tiles of one 64-token pair back to back
        const int mp = 8 * (r / (QE_D / 128)) + x;
        if (mp >= (T + 63) / 64) return;
        shdn_tile64(hhl, T, Wsd, sd, mp, r % (QE_D / 128), (uint8_t *)&sm.s);
        return;
    }
    r -= nshx;
    const int rgb_n = (QE_D / 128) / dn.dn_rgw;
    if (r < nix * rgb_n) dn_unit_at<true>(dn, x + 8 * (r / rgb_n), r % rgb_n, sm.d);
}

hipError_t qe_launch_router_shgu(const QeLayerPtrs &L, const QeScratch &S, int T, hipStream_t st) {
    const int nr = RS_NT * ((T + 63) / 64) * RT_SPLIT, ns = 8 * RS_JT * (((T + 31) / 32 + 7) / 8);
    if (T >= QE_RS_SPLIT_T) {
        k_router<<<nr, 256, 0, st>>>(S.xn, T, L.router, S.rpart);
        k_shgu<<<64 * (((T + 63) / 64 + 7) / 8), 256, 0, st>>>(S.xhl, T, L.sh_gu, (_Float16 *)S.shgu);
    } else {
        k_router_shgu<<<nr + ns, 256, 0, st>>>(S.xn, S.xhl, T, L.router, L.sh_gu, S.rpart, (_Float16 *)S.shgu);
    }
    return hipGetLastError();
}

#ifndef QE_DN_RGW4_T
#define QE_DN_RGW4_T 256
#endif
#ifndef QE_DN_RGW2_T
#define QE_DN_RGW2_T 256
#endif
hipError_t qe_launch_expert_mfma(const QeLayerPtrs &L, const QeScratch &S, int T, hipStream_t st) {
    const int np = T * QE_K_USED;
    GemmTileArgs g{};
    g.arena = L.arena; g.pairs = S.pairs; g.items = S.items; g.n_items = S.n_items; g.wts = S.wts;
    g.aq = S.xqp; g.a_bytes = T * QE_D; g.as = S.xs; g.a_row_div = QE_K_USED; g.hq = S.hqp; g.hs = S.hs;
    const bool fused = T >= QE_FUSE_T_MIN && T < QE_FUSE_T && S.item_done;
    if (fused) {
        g.item_done = S.item_done; g.err = S.err; g.err_val = S.err_val; g.spin_cap = S.spin_cap;
        g.wait_extra = S.wait_extra;
    } else {
        k_expert_gu<<<expert_max_wg<true>(np), 256, 0, st>>>(g);
    }
    GemmTileArgs d = g;
    d.aq = S.hqp; d.a_bytes = np * QE_FF_EXP; d.as = S.hs; d.a_row_div = 1; d.yp = S.yp;
    // row groups per down workgroup: fewer, longer workgroups where the items
    // alone fill the CUs several times over
    // (4 from 256 tokens in separate launches: measured best at 512 and 8192; fused,
    // shorter down workgroups drain the tail sooner: 1 below 512 tokens, then 2)
    d.dn_rgw = fused ? (T < 512 ? 1 : 2) : T >= QE_DN_RGW4_T ? 4 : T >= QE_DN_RGW2_T ? 2 : 1;
    const int nsh = 8 * (QE_D / 128) * (((T + 63) / 64 + 7) / 8);
    const int nr = dn_max_wg(np, d.dn_rgw); // a multiple of 8: shared tiles start on XCD 0
    if (fused) {
        // per XCD at most: 16 gate/up and rgb_n down workgroups for each of its items, and its shared tiles
        const int ix = ((np / (QE_MFMA_MC / 2 + 1) + 1 + QE_N_EXPERT) + 7) / 8, rgb_n = (QE_D / 128) / d.dn_rgw;
        k_expert_gudn<<<8 * ((16 + rgb_n) * ix + nsh / 8), 256, 0, st>>>(g, d, nsh / 8, (const _Float16 *)S.shgu, T,
                                                                          L.sh_dn, S.sd);
    } else
        k_expert_dn<<<nr + nsh, 256, 0, st>>>(d, nr, (const _Float16 *)S.shgu, T, L.sh_dn, S.sd);
    return hipGetLastError();
}
