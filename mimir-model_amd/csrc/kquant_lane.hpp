// Per-lane decode of Q4_K and Q6_K blocks for the 8-bit GEMV kernels: a
// group of eight lanes shares one 256-element block; each helper gives one
// lane its quants (as packed bytes for v_dot4_i32_i8), scales and the
// activation offsets it multiplies. Integer results are exact.
#pragma once

#include "mimg_device.hpp"

namespace mimg {

// One lane's share of a Q4_K block: lane l holds quant bytes 16l..16l+15 of
// the block, i.e. chunk c = l/2, elements 64c+16h+[0,16) (low nibbles,
// sub-block 2c) and 64c+32+16h+[0,16) (high nibbles, sub-block 2c+1), with
// h = l%2; for the M term it takes sub-block l.
struct Q4KLane {
    uint32_t lo[4], hi[4];
    int scl, sch, mm, yoff;
    float d, dmin;
};

__device__ __forceinline__ Q4KLane q4k_lane(const u32x4& hdr, const u32x4& qv, int l) {
    Q4KLane w;
    const Q4KScales s = q4k_scales(hdr.y, hdr.z, hdr.w);
    const int c = l >> 1, h = l & 1;
    w.scl = (int)byte_of(s.sc, 2 * c);
    w.sch = (int)byte_of(s.sc, 2 * c + 1);
    w.mm = (int)byte_of(s.m, l);
    w.d = f16_to_f32(hdr.x & 0xFFFFu);
    w.dmin = f16_to_f32(hdr.x >> 16);
    w.yoff = 64 * c + 16 * h;
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w.lo[k] = q[k] & 0x0F0F0F0Fu;
        w.hi[k] = (q[k] >> 4) & 0x0F0F0F0Fu;
    }
    return w;
}

// The lane's part of S: sc_2c * sum(lo*y) + sc_2c+1 * sum(hi*y) (exact).
__device__ __forceinline__ int q4k_part(const Q4KLane& w, const u32x4& ya, const u32x4& yh) {
    int dl = sdot4(w.lo[0], ya.x, 0);
    dl = sdot4(w.lo[1], ya.y, dl);
    dl = sdot4(w.lo[2], ya.z, dl);
    dl = sdot4(w.lo[3], ya.w, dl);
    int dh = sdot4(w.hi[0], yh.x, 0);
    dh = sdot4(w.hi[1], yh.y, dh);
    dh = sdot4(w.hi[2], yh.z, dh);
    dh = sdot4(w.hi[3], yh.w, dh);
    // |dl|, |dh| <= 16*15*128 and the scales are 6-bit: 24-bit multiplies
    // (full rate) are exact.
    return __mul24(w.scl, dl) + __mul24(w.sch, dh);
}

// Raw loads of one lane's share of a Q6_K block (2-byte aligned blocks):
// lane l = 4h + p takes ql bytes 64h+16p..+16 (elements eL..eL+15 in their
// low nibbles and eH = eL+64.. in their high nibbles, eL = 128h+32(p/2)+16(p%2)),
// the qh bytes 32h+16(p%2)..+16 and the block's scales and d. The 16-byte
// runs are kept as the five aligned dwords that hold them (both runs share
// the block's misalignment); q6k_lane shifts them into place, so nothing
// here waits for the loads to land.
struct Q6KRaw {
    uint32_t ql[5], qh[5];
    int scl, sch;
    uint32_t dbits, shift;
};

// Seven loads per lane: ql and qh as 5 aligned dwords each, the two int8
// scales of the lane's runs of 16 (sc[8h+idx] and sc[8h+idx+4], idx =
// 2(p/2)+p%2) and d.
__device__ __forceinline__ Q6KRaw q6k_load(const uint8_t* blk, int l) {
    const int h = l >> 2, p = l & 3, idx = 2 * (p >> 1) + (p & 1);
    Q6KRaw r;
    const uint32_t* a = (const uint32_t*)__builtin_align_down(blk + 64 * h + 16 * p, 4);
    const uint32_t* c = (const uint32_t*)__builtin_align_down(blk + 128 + 32 * h + 16 * (p & 1), 4);
    const u32x4a4 av = *(const u32x4a4*)a, cv = *(const u32x4a4*)c;
    r.ql[0] = av.x, r.ql[1] = av.y, r.ql[2] = av.z, r.ql[3] = av.w, r.ql[4] = a[4];
    r.qh[0] = cv.x, r.qh[1] = cv.y, r.qh[2] = cv.z, r.qh[3] = cv.w, r.qh[4] = c[4];
    r.shift = (uint32_t)((uintptr_t)blk & 3);
    r.scl = (int)(int8_t)blk[192 + 8 * h + idx];
    r.sch = (int)(int8_t)blk[196 + 8 * h + idx];
    r.dbits = load_u16(blk + 208);
    return r;
}

// The same seven loads from base + off, with base 4-byte aligned and off a
// 32-bit offset (the compiler addresses them as an SGPR base plus one VGPR
// offset each, with the constant parts as immediates).
__device__ __forceinline__ Q6KRaw q6k_load_at(const uint8_t* base, uint32_t off, int l) {
    const uint32_t h = (uint32_t)l >> 2, p = (uint32_t)l & 3, idx = 2 * (p >> 1) + (p & 1);
    Q6KRaw r;
    const uint32_t oa = (off + 64 * h + 16 * p) & ~3u, oc = (off + 128 + 32 * h + 16 * (p & 1)) & ~3u;
    const u32x4a4 av = *(const u32x4a4*)(base + oa), cv = *(const u32x4a4*)(base + oc);
    r.ql[0] = av.x, r.ql[1] = av.y, r.ql[2] = av.z, r.ql[3] = av.w, r.ql[4] = *(const uint32_t*)(base + oa + 16);
    r.qh[0] = cv.x, r.qh[1] = cv.y, r.qh[2] = cv.z, r.qh[3] = cv.w, r.qh[4] = *(const uint32_t*)(base + oc + 16);
    r.shift = off & 3;
    const uint32_t os = off + 8 * h + idx;
    r.scl = (int)*(const int8_t*)(base + os + 192);
    r.sch = (int)*(const int8_t*)(base + os + 196);
    r.dbits = *(const uint16_t*)(base + off + 208);
    return r;
}

struct Q6KLane {
    uint32_t vl[4], vh[4];
    int scl, sch, eL;
    float d;
};

__device__ __forceinline__ Q6KLane q6k_lane(const Q6KRaw& r, int l) {
    const int h = l >> 2, p = l & 3, pp = p >> 1, p1 = p & 1;
    Q6KLane w;
    w.scl = r.scl;
    w.sch = r.sch;
    w.d = f16_to_f32(r.dbits);
    w.eL = 128 * h + 32 * pp + 16 * p1;
    const int shL = 2 * pp, shH = 4 + 2 * pp;
    uint32_t qlw[4], qhw[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        qlw[k] = __builtin_amdgcn_alignbyte(r.ql[k + 1], r.ql[k], r.shift);
        qhw[k] = __builtin_amdgcn_alignbyte(r.qh[k + 1], r.qh[k], r.shift);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w.vl[k] = (qlw[k] & 0x0F0F0F0Fu) | (((qhw[k] >> shL) & 0x03030303u) << 4);
        w.vh[k] = ((qlw[k] >> 4) & 0x0F0F0F0Fu) | (((qhw[k] >> shH) & 0x03030303u) << 4);
    }
    return w;
}

// The lane's part of S: sc_L*(sum(q*y) - 32*sum(y)) + sc_H*(...) over its
// two runs of 16 (exact); ysL/ysH are the runs' activation sums.
__device__ __forceinline__ int q6k_part(const Q6KLane& w, const u32x4& ya, const u32x4& yh, int ysL, int ysH) {
    int dl = sdot4(w.vl[0], ya.x, 0);
    dl = sdot4(w.vl[1], ya.y, dl);
    dl = sdot4(w.vl[2], ya.z, dl);
    dl = sdot4(w.vl[3], ya.w, dl);
    int dh = sdot4(w.vh[0], yh.x, 0);
    dh = sdot4(w.vh[1], yh.y, dh);
    dh = sdot4(w.vh[2], yh.z, dh);
    dh = sdot4(w.vh[3], yh.w, dh);
    // |dl - 32*ysL| <= 16*63*128 + 32*16*128 < 2^23 and the scales are int8:
    // 24-bit multiplies (full rate) are exact.
    return __mul24(w.scl, dl - 32 * ysL) + __mul24(w.sch, dh - 32 * ysH);
}

// One group's share of the activation for one block: Q4_K ya/yh = the 16
// quants of each of its two runs, xs the sum of its sub-block; Q6_K ya/yh
// and the two runs' sums ysL/ysH. dx is the block's activation scale.
struct ActLane {
    u32x4 ya, yh;
    int sa, sb;
    float dx;
};

template <uint32_t DT>
__device__ __forceinline__ ActLane act_lane(const int8_t* q, const int16_t* s16, const float* d32, int64_t K, int m,
                                           int b, int l) {
    const int64_t R32 = K / 32, R16 = K / 16;
    const int8_t* yb = q + m * K + (uint32_t)(b * 256);
    ActLane a;
    if constexpr (DT == DT_Q4_K) {
        const int yoff = 64 * (l >> 1) + 16 * (l & 1);
        a.ya = *(const u32x4*)(yb + yoff);
        a.yh = *(const u32x4*)(yb + yoff + 32);
        a.sa = s16[m * R32 + 8 * b + l];
        a.sb = 0;
    } else {
        const int eL = 128 * (l >> 2) + 32 * ((l & 3) >> 1) + 16 * (l & 1);
        a.ya = *(const u32x4*)(yb + eL);
        a.yh = *(const u32x4*)(yb + eL + 64);
        const int16_t* ys = s16 + m * R16 + 16 * b;
        a.sa = ys[eL >> 4];
        a.sb = ys[(eL + 64) >> 4];
    }
    a.dx = d32[m * R32 + 8 * b];
    return a;
}

// The exact (S, M) of one (row, block) pair for one activation row and the
// two f32 scale products, as the pair table holds them.
template <uint32_t DT>
__device__ __forceinline__ i32x4 pair_part(const u32x4& hdr, const u32x4& qv, const Q6KRaw& raw, const ActLane& a,
                                           int l) {
    i32x4 v;
    if constexpr (DT == DT_Q4_K) {
        const Q4KLane w = q4k_lane(hdr, qv, l);
        v.x = group8_sum(q4k_part(w, a.ya, a.yh));
        v.y = group8_sum(w.mm * a.sa);
        v.z = __float_as_int(w.d * a.dx);
        v.w = __float_as_int(w.dmin * a.dx);
    } else {
        const Q6KLane w = q6k_lane(raw, l);
        v.x = group8_sum(q6k_part(w, a.ya, a.yh, a.sa, a.sb));
        v.y = 0;
        v.z = __float_as_int(w.d * a.dx);
        v.w = 0;
    }
    return v;
}

}  // namespace mimg
