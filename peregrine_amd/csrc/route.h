// route.h — the greedy top-k router of one token on one wavefront, shared
// by the router kernels and the one-token gate/up prologue.
#pragma once

#include "common.h"

namespace phip {

// ---------------------------------------------------------------------------
// Device router for the BASELINE configs: greedy top-k over the logits (strict
// >, ties to the lowest index — the loop of peregrine-model/src/router.rs:97-118)
// then w_j = exp(l_j - l_0) / sum_j exp(l_j - l_0) summed in selection order.
// One wavefront per token.
// ---------------------------------------------------------------------------
// (value desc, index asc) maximum across the wavefront, returned uniform.
// DPP exchanges inside each row of 16 lanes (quad swaps, half-row and row
// mirrors leave all 16 lanes agreeing), then the four row results are read
// as scalars.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float &v, int &i) {
    const float ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
    argmax_dpp<0xB1>(v, i);    // quad_perm [1,0,3,2]
    argmax_dpp<0x4E>(v, i);    // quad_perm [2,3,0,1]
    argmax_dpp<0x141>(v, i);   // row_half_mirror
    argmax_dpp<0x140>(v, i);   // row_mirror
    float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
        const int ri = __builtin_amdgcn_readlane(i, r);
        if (rv > bv || (rv == bv && ri < bi)) {
            bv = rv;
            bi = ri;
        }
    }
    v = bv;
    i = bi;
}

// (value desc, index asc) as one unsigned 64-bit key: the high word orders
// floats as integers (sign-folded, -0 folded onto +0), the low word is the
// complemented index, so a larger key is a larger value or, at equal values,
// a lower index. 0 marks "not a candidate" (NaN, -inf, padding, retired).
__device__ __forceinline__ uint64_t route_key(float v, int e) {
    if (!(v > -INFINITY)) return 0;
    const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ float route_key_value(uint64_t key) {
    const uint32_t ord = (uint32_t)(key >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}
__device__ __forceinline__ int route_key_index(uint64_t key) { return (int)(0xFFFFFFFFu - (uint32_t)key); }

// max(v, v from the DPP-selected lane); lanes the pattern does not feed keep v
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t u32_max_dpp(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROW_MASK, 0xF, false);
    return o > v ? o : v;
}
// wavefront maximum, uniform: quad swaps, half-row and row mirrors give every
// row its maximum, the row broadcasts carry rows 0-2 into row 3, and lane 63
// is read as a scalar. Branch-free.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = u32_max_dpp<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = u32_max_dpp<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = u32_max_dpp<0x141, 0xF>(v);   // row_half_mirror
    v = u32_max_dpp<0x140, 0xF>(v);   // row_mirror
    v = u32_max_dpp<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v = u32_max_dpp<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

template <int PER>
__device__ __forceinline__ void sort_keys_desc(uint64_t (&kv)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; i++)
#pragma unroll
        for (int j = PER - 1; j > i; j--) {
            const uint64_t a = kv[j - 1], b = kv[j];
            kv[j - 1] = a > b ? a : b;
            kv[j] = a > b ? b : a;
        }
}

// The greedy selection of one token on one wavefront: k rounds, each picking
// the largest remaining logit, ties to the lowest index (the loop of
// peregrine-model/src/router.rs:97-118). A lane holds logits e = lane + 64*j
// as keys, sorted so its head is its largest. A round reduces the heads' high
// words (the values) across the wavefront; when several lanes hold that value
// the low words (complemented indices) decide. The owner then pops its head.
// NaN and -inf never qualify, so fewer than k valid logits leave the
// remaining slots empty. Lane kk returns the kk-th pick's key in mykey; kept
// and first (the top key) are uniform.
template <int PER>
__device__ __forceinline__ void route_select(const float *l, int E, int k, uint64_t &mykey, int &kept,
                                             uint64_t &first) {
    const int lane = threadIdx.x & 63;
    uint64_t kv[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane + 64 * j;
        kv[j] = e < E ? route_key(l[e], e) : 0;
    }
    sort_keys_desc<PER>(kv);
    mykey = 0;
    first = 0;
    kept = 0;
    for (int kk = 0; kk < k; kk++) {
        const uint32_t hv = (uint32_t)(kv[0] >> 32);
        const uint32_t mv = wave_max_u32(hv);
        if (mv == 0) break;   // uniform: nothing valid remains
        const uint64_t tied = __ballot(hv == mv);
        uint32_t lo;
        if ((tied & (tied - 1)) == 0) {   // one lane holds the maximum value
            lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kv[0], __builtin_ctzll(tied));
        } else {
            lo = wave_max_u32(hv == mv ? (uint32_t)kv[0] : 0u);
        }
        const uint64_t best = ((uint64_t)mv << 32) | lo;
        if (lane == kk) mykey = best;
        if (kk == 0) first = best;
        if (kv[0] == best) {   // the owner pops its head (keys are unique)
#pragma unroll
            for (int j = 0; j + 1 < PER; j++) kv[j] = kv[j + 1];
            kv[PER - 1] = 0;
        }
        kept++;
    }
}

// Slot ids and softmax weights from a selection: empty slots get id 0 and
// weight 0; w_j = exp(l_j - l_0) / sum_j exp(l_j - l_0), the sum taken in
// selection order. desc/row_desc (optional): copy the chosen experts'
// descriptors per slot.
__device__ __forceinline__ void route_weights(uint64_t mykey, int kept, uint64_t first, int k, int *ids, float *w,
                                              const ExpertDesc *desc, ExpertDesc *row_desc) {
    const int lane = threadIdx.x & 63;
    const float l0 = route_key_value(first);
    const float myex = lane < kept ? expf_glibc(__fsub_rn(route_key_value(mykey), l0)) : 0.0f;
    float z = 0.0f;
    for (int kk = 0; kk < kept; kk++)
        z = __fadd_rn(z, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myex), kk)));
    if (lane < k) {
        const bool ok = lane < kept;
        const int id = ok ? route_key_index(mykey) : 0;
        ids[lane] = id;
        w[lane] = ok ? __fdiv_rn(myex, z) : 0.0f;
        if (row_desc) row_desc[lane] = desc[id];
    }
}

// One wavefront routes one token: selection, then weights.
template <int PER>
__device__ void route_token(const float *l, int E, int k, int *ids, float *w, const ExpertDesc *desc,
                            ExpertDesc *row_desc) {
    uint64_t mykey, first;
    int kept;
    route_select<PER>(l, E, k, mykey, kept, first);
    route_weights(mykey, kept, first, k, ids, w, desc, row_desc);
}

// Elements 8*gi .. 8*gi+7 of an activation row (zero past K); vec: K % 8 == 0
// and the row is 16-byte aligned, so a group is two 16-byte loads.
__device__ __forceinline__ void load_group8(const float *x, int gi, int K, bool vec, float (&v)[8]) {
    const auto *xg = gptr(x);
    if (vec) {
        if (gi * 8 < K) {
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 a = *(const __attribute__((address_space(1))) f4 *)(xg + gi * 8);
            const f4 b = *(const __attribute__((address_space(1))) f4 *)(xg + gi * 8 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = gi * 8 + j < K ? xg[gi * 8 + j] : 0.0f;
    }
}

// maximum over the four lanes of a quad (one 32-block), every lane agreeing
__device__ __forceinline__ float quad_max(float m) {
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    return m;
}

// qrow_i8 (peregrine-kernels/src/quant.rs:14-33) of one 32-element block held
// by four consecutive lanes, eight elements each; every lane returns the
// block scale and its eight codes packed in the device byte order (perm8:
// even elements in the low dword, odd in the high one).
__device__ __forceinline__ float quant_group8(const float (&v)[8], float m_in, uint2 &packed) {
    float sc = __fdiv_rn(m_in, 127.0f);
    if (sc < 1e-12f) sc = 1e-12f;
    const float inv = __fdiv_rn(1.0f, sc);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)rintf(__fmul_rn(v[j], inv));
        if (j & 1) hi |= b << (8 * (j >> 1));
        else lo |= b << (8 * (j >> 1));
    }
    packed = make_uint2(lo, hi);
    return sc;
}

// ACT_B32 quantisation (quant.rs:14-33 per 32-block) of the 8-element groups
// [g_lo, g_hi) of one row: thread t of nt cooperating threads takes groups
// g_lo + t, g_lo + t + nt, ...; a 32-block is four consecutive threads, so
// g_lo and nt are multiples of 4 and quads of threads are quad-aligned lanes.
// Codes go out packed (8 bytes per group, device order), scales once per block.
__device__ __forceinline__ void quant_row_b32(const float *x, int K, int Kp, int8_t *q, float *sc, int g_lo, int g_hi,
                                              int t, int nt) {
    const int ngr = Kp >> 3;
    const bool vec = (K & 7) == 0 && ((uintptr_t)x & 15) == 0;
    for (int base = g_lo; base < g_hi; base += nt) {
        const int gi = base + t;
        float v[8];
        load_group8(x, gi < g_hi ? gi : ngr, K, vec, v);   // past the range: zeros
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(v[j]));
        m = quad_max(m);
        uint2 pk;
        const float s = quant_group8(v, m, pk);
        if (gi < g_hi) {
            *(uint2 *)(q + (size_t)gi * 8) = pk;
            if ((gi & 3) == 0) sc[gi >> 2] = s;
        }
    }
}

}  // namespace phip
