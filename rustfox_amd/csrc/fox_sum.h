// fox_sum.h -- float sums in a fixed order for the attention kernels: the
// one-add-at-a-time chain fed from LDS (chain_lds16, chain_quads: the value
// sums of src/ops.c and forward.c, one chain per lane) and the softmax sum
// of src/ops.c:31-33 (sum += e_j for j = 0, 1, ..., each add rounded to
// nearest even, in that order) formed by a whole wave a run of elements at a
// time (sum_in_order), with the chain's result.
#pragma once

#include "fox_gemv_dev.h"

// acc + x_0 + ... + x_{4n-1} over float4 p[0 .. n) of LDS, in order.
// A dependent add chain is bound by the wave's instruction issue, so its
// operands must arrive ahead of it: in chain_lds16 two banks of eight quads
// (v64-v95, v96-v127) alternate, one bank's reads in flight while the other
// bank's 32 adds run (software pipelining across the loop, which the
// compiler does not do: compiled from C, each group's reads are issued
// after the previous group's adds and their latency is paid every time).
// LDS returns a wave's reads in order, so lgkmcnt(8) after a bank's reads
// means the bank before is in (earlier outstanding scalar loads only make
// that wait stricter).  The asm ends with lgkmcnt(0).  q is the lane's own
// address; ng >= 1 groups of 16 quads.
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

__device__ __forceinline__ float chain_lds16(float acc, const float4 *q, int ng)
{
    uint32_t p = lds_addr(q);
    int i = ng;
    asm volatile(
        "ds_read_b128 v[64:67], %[p] offset:0\n"
        "ds_read_b128 v[68:71], %[p] offset:16\n"
        "ds_read_b128 v[72:75], %[p] offset:32\n"
        "ds_read_b128 v[76:79], %[p] offset:48\n"
        "ds_read_b128 v[80:83], %[p] offset:64\n"
        "ds_read_b128 v[84:87], %[p] offset:80\n"
        "ds_read_b128 v[88:91], %[p] offset:96\n"
        "ds_read_b128 v[92:95], %[p] offset:112\n"
        "1:\n"
        "ds_read_b128 v[96:99], %[p] offset:128\n"
        "ds_read_b128 v[100:103], %[p] offset:144\n"
        "ds_read_b128 v[104:107], %[p] offset:160\n"
        "ds_read_b128 v[108:111], %[p] offset:176\n"
        "ds_read_b128 v[112:115], %[p] offset:192\n"
        "ds_read_b128 v[116:119], %[p] offset:208\n"
        "ds_read_b128 v[120:123], %[p] offset:224\n"
        "ds_read_b128 v[124:127], %[p] offset:240\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[acc], %[acc], v64\n"
        "v_add_f32 %[acc], %[acc], v65\n"
        "v_add_f32 %[acc], %[acc], v66\n"
        "v_add_f32 %[acc], %[acc], v67\n"
        "v_add_f32 %[acc], %[acc], v68\n"
        "v_add_f32 %[acc], %[acc], v69\n"
        "v_add_f32 %[acc], %[acc], v70\n"
        "v_add_f32 %[acc], %[acc], v71\n"
        "v_add_f32 %[acc], %[acc], v72\n"
        "v_add_f32 %[acc], %[acc], v73\n"
        "v_add_f32 %[acc], %[acc], v74\n"
        "v_add_f32 %[acc], %[acc], v75\n"
        "v_add_f32 %[acc], %[acc], v76\n"
        "v_add_f32 %[acc], %[acc], v77\n"
        "v_add_f32 %[acc], %[acc], v78\n"
        "v_add_f32 %[acc], %[acc], v79\n"
        "v_add_f32 %[acc], %[acc], v80\n"
        "v_add_f32 %[acc], %[acc], v81\n"
        "v_add_f32 %[acc], %[acc], v82\n"
        "v_add_f32 %[acc], %[acc], v83\n"
        "v_add_f32 %[acc], %[acc], v84\n"
        "v_add_f32 %[acc], %[acc], v85\n"
        "v_add_f32 %[acc], %[acc], v86\n"
        "v_add_f32 %[acc], %[acc], v87\n"
        "v_add_f32 %[acc], %[acc], v88\n"
        "v_add_f32 %[acc], %[acc], v89\n"
        "v_add_f32 %[acc], %[acc], v90\n"
        "v_add_f32 %[acc], %[acc], v91\n"
        "v_add_f32 %[acc], %[acc], v92\n"
        "v_add_f32 %[acc], %[acc], v93\n"
        "v_add_f32 %[acc], %[acc], v94\n"
        "v_add_f32 %[acc], %[acc], v95\n"
        "v_add_u32 %[p], 256, %[p]\n"
        "s_sub_u32 %[i], %[i], 1\n"
        "s_cmp_eq_u32 %[i], 0\n"
        "s_cbranch_scc1 2f\n"
        "ds_read_b128 v[64:67], %[p] offset:0\n"
        "ds_read_b128 v[68:71], %[p] offset:16\n"
        "ds_read_b128 v[72:75], %[p] offset:32\n"
        "ds_read_b128 v[76:79], %[p] offset:48\n"
        "ds_read_b128 v[80:83], %[p] offset:64\n"
        "ds_read_b128 v[84:87], %[p] offset:80\n"
        "ds_read_b128 v[88:91], %[p] offset:96\n"
        "ds_read_b128 v[92:95], %[p] offset:112\n"
        "s_waitcnt lgkmcnt(8)\n"
        "v_add_f32 %[acc], %[acc], v96\n"
        "v_add_f32 %[acc], %[acc], v97\n"
        "v_add_f32 %[acc], %[acc], v98\n"
        "v_add_f32 %[acc], %[acc], v99\n"
        "v_add_f32 %[acc], %[acc], v100\n"
        "v_add_f32 %[acc], %[acc], v101\n"
        "v_add_f32 %[acc], %[acc], v102\n"
        "v_add_f32 %[acc], %[acc], v103\n"
        "v_add_f32 %[acc], %[acc], v104\n"
        "v_add_f32 %[acc], %[acc], v105\n"
        "v_add_f32 %[acc], %[acc], v106\n"
        "v_add_f32 %[acc], %[acc], v107\n"
        "v_add_f32 %[acc], %[acc], v108\n"
        "v_add_f32 %[acc], %[acc], v109\n"
        "v_add_f32 %[acc], %[acc], v110\n"
        "v_add_f32 %[acc], %[acc], v111\n"
        "v_add_f32 %[acc], %[acc], v112\n"
        "v_add_f32 %[acc], %[acc], v113\n"
        "v_add_f32 %[acc], %[acc], v114\n"
        "v_add_f32 %[acc], %[acc], v115\n"
        "v_add_f32 %[acc], %[acc], v116\n"
        "v_add_f32 %[acc], %[acc], v117\n"
        "v_add_f32 %[acc], %[acc], v118\n"
        "v_add_f32 %[acc], %[acc], v119\n"
        "v_add_f32 %[acc], %[acc], v120\n"
        "v_add_f32 %[acc], %[acc], v121\n"
        "v_add_f32 %[acc], %[acc], v122\n"
        "v_add_f32 %[acc], %[acc], v123\n"
        "v_add_f32 %[acc], %[acc], v124\n"
        "v_add_f32 %[acc], %[acc], v125\n"
        "v_add_f32 %[acc], %[acc], v126\n"
        "v_add_f32 %[acc], %[acc], v127\n"
        "s_branch 1b\n"
        "2:\n"
        "s_waitcnt lgkmcnt(0)\n"
        "v_add_f32 %[acc], %[acc], v96\n"
        "v_add_f32 %[acc], %[acc], v97\n"
        "v_add_f32 %[acc], %[acc], v98\n"
        "v_add_f32 %[acc], %[acc], v99\n"
        "v_add_f32 %[acc], %[acc], v100\n"
        "v_add_f32 %[acc], %[acc], v101\n"
        "v_add_f32 %[acc], %[acc], v102\n"
        "v_add_f32 %[acc], %[acc], v103\n"
        "v_add_f32 %[acc], %[acc], v104\n"
        "v_add_f32 %[acc], %[acc], v105\n"
        "v_add_f32 %[acc], %[acc], v106\n"
        "v_add_f32 %[acc], %[acc], v107\n"
        "v_add_f32 %[acc], %[acc], v108\n"
        "v_add_f32 %[acc], %[acc], v109\n"
        "v_add_f32 %[acc], %[acc], v110\n"
        "v_add_f32 %[acc], %[acc], v111\n"
        "v_add_f32 %[acc], %[acc], v112\n"
        "v_add_f32 %[acc], %[acc], v113\n"
        "v_add_f32 %[acc], %[acc], v114\n"
        "v_add_f32 %[acc], %[acc], v115\n"
        "v_add_f32 %[acc], %[acc], v116\n"
        "v_add_f32 %[acc], %[acc], v117\n"
        "v_add_f32 %[acc], %[acc], v118\n"
        "v_add_f32 %[acc], %[acc], v119\n"
        "v_add_f32 %[acc], %[acc], v120\n"
        "v_add_f32 %[acc], %[acc], v121\n"
        "v_add_f32 %[acc], %[acc], v122\n"
        "v_add_f32 %[acc], %[acc], v123\n"
        "v_add_f32 %[acc], %[acc], v124\n"
        "v_add_f32 %[acc], %[acc], v125\n"
        "v_add_f32 %[acc], %[acc], v126\n"
        "v_add_f32 %[acc], %[acc], v127\n"
        : [acc] "+&v"(acc), [p] "+&v"(p), [i] "+&s"(i)
        :
        : "v64", "v65", "v66", "v67", "v68", "v69", "v70", "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83", "v84", "v85", "v86", "v87", "v88", "v89", "v90", "v91", "v92", "v93", "v94", "v95", "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122", "v123", "v124", "v125", "v126", "v127", "scc", "memory");
    return acc;
}

// acc + x_0 + ... + x_{4n-1} over float4 p[0 .. n) of LDS, in order
__device__ __forceinline__ float chain_quads(float acc, const float4 *p, int n)
{
    const int ng = n >> 4;
    if (ng > 0) acc = chain_lds16(acc, p, ng);
    for (int i = ng << 4; i < n; i++) {
        const float4 v = p[i];
        acc = acc + v.x; acc = acc + v.y; acc = acc + v.z; acc = acc + v.w;
    }
    return acc;
}

// inclusive prefix sum of v over the wave's lanes (lane l: v_0 + ... + v_l)
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v)
{
    v += dpp_t<0x111, 0xF>(0u, v);       // row_shr:1 (zero shifted in)
    v += dpp_t<0x112, 0xF>(0u, v);       // row_shr:2
    v += dpp_t<0x114, 0xF>(0u, v);       // row_shr:4
    v += dpp_t<0x118, 0xF>(0u, v);       // row_shr:8: rows of 16 done
    v += dpp_t<0x142, 0xA>(0u, v);       // row_bcast:15 into rows 1 and 3
    v += dpp_t<0x143, 0xC>(0u, v);       // row_bcast:31 into rows 2 and 3
    return v;
}

__device__ __forceinline__ float uniform_f(float x)
{
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// element k of a 4-vector (k uniform)
__device__ __forceinline__ float f4_at(const float __attribute__((ext_vector_type(4))) &v, int k)
{
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// acc + e[0] + e[1] + ... + e[n-1], each add rounded to nearest even, in that
// order, over e in LDS (16-byte aligned).  The whole wave calls it, every
// lane returns the sum.  e is read SUM_CHUNK floats at a time, so LDS up to
// SUM_CHUNK floats past e + n must lie inside the workgroup's allocation
// (those values are not used).
//
// While the running sum s is a normal float in a binade [2^E, 2^(E+1)),
// every float there is a multiple of u = 2^(E-23), and if s + e stays below
// 2^(E+1) the rounded sum is u (s/u + r) with r = e/u rounded to the nearest
// integer: s/u is an integer, so the rounding of s + e is that of e/u alone
// (but for a tie, e/u ending in exactly one half, which goes to the even
// multiple and so depends on s/u).  Over a run of elements that stays in the
// binade, s/u therefore grows by integer prefix sums of the r_j, which the
// wave forms for SUM_CHUNK elements at once (four per lane and a lane
// scan).  An event ends a run: the first element whose rounded sum reaches
// 2^(E+1) (its exact sum may lie above, where the floats are 2u apart), a
// tie, an element that is infinite or NaN or whose e/u reaches 2^23.  At an
// event s becomes u times the integer sum before the element (exact: at
// most 2^24 u = 2^(E+1)) and the element is added with the hardware's own
// add, as the one-element-at-a-time chain does; the runs resume after it.  A
// sum that is zero, subnormal, infinite or NaN, and a chunk holding a
// negative element, take the elements one at a time the same way.  The
// result is that chain's, bit for bit, but for a NaN sum, which is returned
// as soon as it appears (any NaN: whatever is added after it, the chain's
// sum stays NaN, and the softmax then uses 1 in place of 1/sum, so which NaN
// it is never shows).
//
// A run of 256 elements costs about 700-900 clocks (the lane scan and the
// scalar hand-overs are one dependent sequence), an event as much: against
// the chain's 6.2 clocks per element it pays where events are rare, that is
// once the sum has grown large against the elements (late in a long context).
#define SUM_CHUNK 256
__device__ __forceinline__ float sum_in_order(float acc, const float *e, int n)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    acc = uniform_f(acc);
    if (n <= 0) return acc;
    // the chunk [c0, c0 + 256) in registers (lane l: c0 + 4l ..), its
    // elements before i and from n on zeroed (they add +0 and make no event);
    // the next chunk in flight (the last one re-read past the end)
    const int clast = (n - 1) & ~255;
    int c0 = 0, i = 0;
    f4v vn = *(const f4v *)(e + 4 * lane), v = vn;
    bool fresh = true, neg = false;
    while (i < n) {                                          // (uniform)
        if (fresh) {
            v = vn;
            vn = *(const f4v *)(e + min(c0 + 256, clast) + 4 * lane);
            const int j = c0 + 4 * lane;
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = j + k < n ? v[k] : 0.0f;
            neg = __builtin_amdgcn_ballot_w64(v[0] < 0.0f || v[1] < 0.0f || v[2] < 0.0f ||
                                              v[3] < 0.0f) != 0;
            fresh = false;
        }
        if (acc != acc) return acc;                         // NaN stays NaN (see below)
        if (neg || !(acc >= 0x1p-126f && acc < INFINITY)) {
            const int d = i - c0;
            acc = uniform_f(acc + read_lane(f4_at(v, d & 3), d >> 2));
            const int j = c0 + 4 * lane;
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = j + k == i ? 0.0f : v[k];
            i++;
        } else {
            const int E = (int)(__float_as_uint(acc) >> 23) - 127;
            const float u = __builtin_ldexpf(1.0f, E - 23);
            const uint32_t N0 = (uint32_t)__builtin_ldexpf(acc, 23 - E);   // [2^23, 2^24)
            const uint32_t D = (1u << 24) - N0;
            uint32_t r[4];
            bool bad = false;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float f = __builtin_ldexpf(v[k], 23 - E);   // exact (or below 2^-126)
                r[k] = (uint32_t)__builtin_rintf(f);     // (garbage where bad: after the event)
                bad = bad || !(f < 0x1p23f) || __builtin_amdgcn_fractf(f) == 0.5f;
            }
            const uint32_t t = r[0] + r[1] + r[2] + r[3];
            const uint32_t inc = wave_scan_u32(t);
            const uint64_t mc = __builtin_amdgcn_ballot_w64(inc >= D);
            const uint64_t mb = __builtin_amdgcn_ballot_w64(bad);
            if ((mc | mb) == 0) {                            // (uniform)
                acc = uniform_f((float)(N0 + read_lane(inc, 63)) * u);
                i = c0 + 256;
            } else {
                // the first lane with an event, the first event in it and
                // the integer sum before that element
                const int L = (int)__builtin_ctzll(mc | mb);
                uint32_t Pb = inc - t;
                int kk = 3;
#pragma unroll
                for (int k = 3; k >= 0; k--) {
                    uint32_t Pk = inc - t;
                    for (int q = 0; q < k; q++) Pk += r[q];
                    const float f = __builtin_ldexpf(v[k], 23 - E);
                    const bool evk = !(f < 0x1p23f) || __builtin_amdgcn_fractf(f) == 0.5f ||
                                     Pk + r[k] >= D;
                    if (evk) {
                        kk = k;
                        Pb = Pk;
                    }
                }
                const int k = read_lane(kk, L);
                acc = (float)(N0 + read_lane(Pb, L)) * u;
                acc = uniform_f(acc + read_lane(f4_at(v, k), L));
                const int q = c0 + 4 * L + k;
                i = q + 1;
                const int j = c0 + 4 * lane;
#pragma unroll
                for (int kq = 0; kq < 4; kq++) v[kq] = j + kq <= q ? 0.0f : v[kq];
            }
        }
        if (i >= c0 + 256) {
            c0 += 256;
            fresh = true;
        }
    }
    return acc;
}
