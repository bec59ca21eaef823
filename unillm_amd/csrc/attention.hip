// attention.hip -- attention with a KV cache in HBM: decode steps (m H / KVH <= 16 new
// query rows a kv head) and prompt-length calls (any m; the tiled kernels further down).
//
// The cache's filled length is device state (the handle's `state`): the first kernel
// of a call reads it and publishes it for the second, which advances it by m.  So the
// kernels never take the length from the host, and a call captured into a HIP graph
// appends at a new position every replay.
//
// What it computes: LlamaAttention::forward_with_cache after the projections
// (crates/runtime/src/models_v2/llama.rs:1044-1150): RoPE on q and k at the
// positions len .. len + m - 1 (apply_rope_with_offset, llama.rs:827-883: the
// half-split rotation, inv_freq and angles in f32), k and v appended to the
// layer's cache (LayerKVCache::append, crates/runtime/src/kv_cache.rs:91-130),
// then softmax(q k^T / sqrt(hd) + causal mask) v for every head, head h reading
// kv head h / (H / KVH) (the reference expands k, v to all heads before
// caching; the cache here keeps the KVH heads, which is the same arithmetic).
// Bound: HBM -- the cached K and V are read once per step (2 KVH len hd 4 bytes,
// f32 like the reference's cache).
//
// Two kernels on the caller's stream.  attn_decode_kernel: a workgroup per (kv
// head g, chunk c of C positions), 256 threads:
//   1. the Q = m G queries of kv head g (the m tokens times the G = H / KVH heads
//      of the group): RoPE at position len + t, times 1 / sqrt(hd), into LDS;
//   2. the new positions len .. len + m - 1 inside this chunk: k rotated and v
//      into LDS, and appended to the cache (each position lies in exactly one
//      chunk, so exactly one workgroup writes it; the scores read these
//      positions from LDS, never back from the cache);
//   3. scores: LP = hd / 8 lanes per position, each with 8 dimensions of k and of
//      every query in registers (256 / LP positions at a time), the dot reduced
//      over the LP lanes by DPP; causal mask; into LDS;
//   4. per query (a wave each), the chunk's max and the exponentials and their sum;
//   5. p v: a float4 of dimensions per thread, positions split over 256 / (hd / 4)
//      thread groups, whose sums meet by lane shuffles within a wave and one LDS
//      pass across the four waves;
//   6. the chunk's (max, sum) pair and o[hd] per query to the workspace.
// attn_merge_kernel: a workgroup per (token, head) merges the chunks by
// log-sum-exp into the output rows [m, H hd].  The kernel boundary makes the
// chunk results of every XCD visible to it.  (Merging in the last workgroup of
// each kv head instead needs an agent-scope release -- an L2 write-back -- in
// every workgroup and serialises the merge on one CU a head: measured 3-9 us
// slower.)
// Everything a step reads from HBM beyond the cache is the m qkv rows and the
// per-chunk results (chunks (hd + 2) floats per query, written and read once).
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <type_traits>

#include "internal.hpp"

namespace unillm {
namespace {

constexpr int kAttnMaxQ = 16;  // queries per kv head in one call: m * H / KVH
constexpr int kThreads = 256;
constexpr int kMaxChunk = 256;   // positions per workgroup
constexpr int kMaxChunks = 512;  // workgroups per kv head (L <= 131072)

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of LP lanes (8, 16 or 32); every lane of a group gets it.
template <int LP>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: quad sums
    v += dpp<0x141>(v);  // row_half_mirror: lane i + lane 7 - i of each 8 -> 8-lane sums
    if constexpr (LP >= 16) v += dpp<0x140>(v);  // row_mirror: lane i + lane 15 - i
    if constexpr (LP >= 32) v += __shfl_xor(v, 16, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_add(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Dynamic LDS (floats): qs[QB][D] | nk[m][D] | nv[m][D] | sp[QB][C] (scores, then
// exponentials) | red[4][QB][D] | stat[QB][2]
// state: the cache's device state ([0] filled length, [1] overflow flag, [2] this
// call's length, published by workgroup (0, 0) for the merge kernel).
template <int D, int QB>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(
    const float* __restrict__ qkv, int m, int H, int KVH, int* __restrict__ state, int C,
    int chunks, float scale, const float* __restrict__ inv_freq, float* __restrict__ kc,
    float* __restrict__ vc, int max_seq, float* __restrict__ part) {
    constexpr int LP = D / 8;             // lanes per position in the score pass
    constexpr int SG = kThreads / LP;     // positions at a time (32, 16, 8)
    constexpr int D4 = D / 4;             // float4 columns in the p v pass
    constexpr int NG = kThreads / D4;     // position groups in the p v pass (16, 8, 4)
    constexpr int HALF = D / 2;
    const int g = blockIdx.x, c = blockIdx.y;
    const int G = H / KVH, Q = m * G;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float* kg = kc + (int64_t)g * max_seq * D;
    const float* vg = vc + (int64_t)g * max_seq * D;

    // score pass: group sg = tid / LP takes positions j0 + sg + SG u (+ UK SG per
    // iteration), lane l8 = tid % LP dimensions 8 l8 .. 8 l8 + 7; p v pass: group
    // pg = tid / D4 takes positions j0 + pg + NG u (+ UV NG per iteration), column
    // c4 = tid % D4.  Cached positions (< len) come from HBM, requested one iteration
    // ahead.  The first iteration's k and v are requested before anything else, the
    // length included: rows clamped into the cache, and a row at or past the filled
    // length is never used (new positions are read from LDS, positions past the
    // chunk's end are masked), so the length's latency and theirs overlap.
    // positions a thread per iteration, 2 of k and 4 of v: the registers leave room for
    // more waves (one query a kv head: 100 VGPRs, five waves a SIMD), and a 32-position
    // chunk is one iteration with no clamped repeats.  Against 4 / 8: the whole
    // Llama-2-7B decode step 1 % faster at L 1024 and L 4096 (KV from HBM), GQA 32/8
    // calls 7-10 % faster; deeper loops (8 / 16) were 8-20 % slower at L 1024
    constexpr int UK = 2, UV = 4;
    const int sg = tid / LP, l8 = tid % LP;
    const int pg = tid / D4, c4 = tid % D4;
    const int j0 = c * C;
    float kA[UK][8], kB[UK][8];
    float4 vA[UV], vB[UV];
#pragma unroll
    for (int u = 0; u < UK; ++u) {
        const float* src = kg + (int64_t)min(j0 + sg + u * SG, max_seq - 1) * D + 8 * l8;
        const float4 a = *reinterpret_cast<const float4*>(src);
        const float4 b = *reinterpret_cast<const float4*>(src + 4);
        kA[u][0] = a.x; kA[u][1] = a.y; kA[u][2] = a.z; kA[u][3] = a.w;
        kA[u][4] = b.x; kA[u][5] = b.y; kA[u][6] = b.z; kA[u][7] = b.w;
    }
#pragma unroll
    for (int u = 0; u < UV; ++u)
        vA[u] = *reinterpret_cast<const float4*>(vg + (int64_t)min(j0 + pg + u * NG, max_seq - 1) * D +
                                                 4 * c4);
    const int len = state[0];
    if (g == 0 && c == 0 && tid == 0) state[2] = len;
    if (len + m > max_seq) return;  // overflow: nothing appended; the merge reports it
    const int j1 = min(j0 + C, len + m);
    const int n = j1 - j0;
    if (n <= 0) {  // a chunk past the filled positions (a grid sized for max_seq): empty
        float* ms = part;
        float* po = part + (int64_t)m * H * chunks * 2;
        for (int i = tid; i < Q * D; i += kThreads) {
            const int qi = i / D, d = i - qi * D;
            const int t = qi / G, e = qi - t * G;
            const int64_t qc = ((int64_t)t * H + g * G + e) * chunks + c;
            if (d == 0) *reinterpret_cast<float2*>(ms + 2 * qc) = make_float2(-INFINITY, 0.0f);
            po[qc * D + d] = 0.0f;
        }
        return;
    }
    const int64_t W = (int64_t)(H + 2 * KVH) * D;  // floats per qkv row
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* qs = sm;
    float* nk = qs + QB * D;
    float* nv = nk + m * D;
    float* sp = nv + m * D;
    float* red = sp + QB * C;
    float* stat = red + 4 * QB * D;
    const int nit_k = (n + UK * SG - 1) / (UK * SG), nit_v = (n + UV * NG - 1) / (UV * NG);
    auto load_k = [&](float (&kr)[UK][8], int it) {
#pragma unroll
        for (int u = 0; u < UK; ++u) {
            const int j = j0 + min(it * UK * SG + sg + u * SG, n - 1);
            const float* src = kg + (int64_t)(j < len ? j : 0) * D + 8 * l8;  // branch-free
            const float4 a = *reinterpret_cast<const float4*>(src);
            const float4 b = *reinterpret_cast<const float4*>(src + 4);
            kr[u][0] = a.x; kr[u][1] = a.y; kr[u][2] = a.z; kr[u][3] = a.w;
            kr[u][4] = b.x; kr[u][5] = b.y; kr[u][6] = b.z; kr[u][7] = b.w;
        }
    };
    auto load_v = [&](float4 (&vr)[UV], int it) {
#pragma unroll
        for (int u = 0; u < UV; ++u) {
            const int j = j0 + min(it * UV * NG + pg + u * NG, n - 1);
            vr[u] = *reinterpret_cast<const float4*>(vg + (int64_t)(j < len ? j : 0) * D + 4 * c4);
        }
    };

    // 1. rotated, scaled queries
    for (int i = tid; i < Q * HALF; i += kThreads) {
        const int qi = i / HALF, p = i - qi * HALF;
        const int t = qi / G, e = qi - t * G;
        const float* x = qkv + t * W + (int64_t)(g * G + e) * D;
        float sn, cs;
        sincosf((float)(len + t) * inv_freq[p], &sn, &cs);
        const float a = x[p], b = x[p + HALF];
        qs[qi * D + p] = (a * cs - b * sn) * scale;
        qs[qi * D + p + HALF] = (a * sn + b * cs) * scale;
    }
    // 2. new positions [nb, j1) of this chunk: k rotated, v copied; into LDS and the cache
    const int nb = max(j0, len);
    for (int i = tid; i < (j1 - nb) * D; i += kThreads) {
        const int j = nb + i / D, d = i % D, t = j - len;
        const float* xk = qkv + t * W + (int64_t)(H + g) * D;
        const float* xv = qkv + t * W + (int64_t)(H + KVH + g) * D;
        const int p = d < HALF ? d : d - HALF;
        float sn, cs;
        sincosf((float)j * inv_freq[p], &sn, &cs);
        const float a = xk[p], b = xk[p + HALF];
        const float kv = d < HALF ? a * cs - b * sn : a * sn + b * cs;
        const float vv = xv[d];
        nk[t * D + d] = kv;
        nv[t * D + d] = vv;
        kc[((int64_t)g * max_seq + j) * D + d] = kv;
        vc[((int64_t)g * max_seq + j) * D + d] = vv;
    }
    __syncthreads();

    // 3. scores (causal mask applied), into sp
    {
        float qr[QB][8];
#pragma unroll
        for (int qi = 0; qi < QB; ++qi) {
            const float4 a = *reinterpret_cast<const float4*>(qs + min(qi, Q - 1) * D + 8 * l8);
            const float4 b = *reinterpret_cast<const float4*>(qs + min(qi, Q - 1) * D + 8 * l8 + 4);
            qr[qi][0] = a.x; qr[qi][1] = a.y; qr[qi][2] = a.z; qr[qi][3] = a.w;
            qr[qi][4] = b.x; qr[qi][5] = b.y; qr[qi][6] = b.z; qr[qi][7] = b.w;
        }
        auto score = [&](float (&kr)[UK][8], int it) {
#pragma unroll
            for (int u = 0; u < UK; ++u) {
                const int jl = it * UK * SG + sg + u * SG;
                const int j = j0 + min(jl, n - 1);
                if (j >= len) {  // a new position: its rotated k is in LDS
                    const float4 a = *reinterpret_cast<const float4*>(nk + (j - len) * D + 8 * l8);
                    const float4 b = *reinterpret_cast<const float4*>(nk + (j - len) * D + 8 * l8 + 4);
                    kr[u][0] = a.x; kr[u][1] = a.y; kr[u][2] = a.z; kr[u][3] = a.w;
                    kr[u][4] = b.x; kr[u][5] = b.y; kr[u][6] = b.z; kr[u][7] = b.w;
                }
#pragma unroll
                for (int qi = 0; qi < QB; ++qi) {
                    float s = 0.0f;
#pragma unroll
                    for (int d = 0; d < 8; ++d) s = fmaf(qr[qi][d], kr[u][d], s);
                    s = group_sum<LP>(s);
                    // lane qi % LP of the group stores query qi's score
                    if (jl < n && qi < Q && qi % LP == l8) {
                        const bool visible = j <= len + qi / G;  // causal
                        sp[qi * C + jl] = visible ? s : -INFINITY;
                    }
                }
            }
        };
        for (int it = 0; it < nit_k; it += 2) {  // wave-uniform trip count
            if (it + 1 < nit_k) load_k(kB, it + 1);
            score(kA, it);
            if (it + 1 < nit_k) {
                if (it + 2 < nit_k) load_k(kA, it + 2);
                score(kB, it + 1);
            }
        }
    }
    // the p v pass's second iteration, requested now (the k registers are free) so
    // its latency passes during the softmax
    if (nit_v > 1) load_v(vB, 1);
    __syncthreads();

    // 4. per query: the chunk's max, exponentials and their sum (a wave per query)
    for (int qi = wv; qi < Q; qi += kThreads / 64) {
        float mx = -INFINITY;
        for (int jl = lane; jl < n; jl += 64) mx = fmaxf(mx, sp[qi * C + jl]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (int jl = lane; jl < n; jl += 64) {
            const float pv = mx == -INFINITY ? 0.0f : expf(sp[qi * C + jl] - mx);
            sp[qi * C + jl] = pv;
            sum += pv;
        }
        sum = wave_add(sum);
        if (lane == 0) {
            stat[2 * qi] = mx;
            stat[2 * qi + 1] = sum;
        }
    }
    __syncthreads();

    // 5. o = p v
    {
        float4 o[QB];
#pragma unroll
        for (int qi = 0; qi < QB; ++qi) o[qi] = make_float4(0.f, 0.f, 0.f, 0.f);
        auto accumulate = [&](float4 (&vr)[UV], int it) {
#pragma unroll
            for (int u = 0; u < UV; ++u) {
                const int jl = it * UV * NG + pg + u * NG;
                if (jl >= n) break;
                const int j = j0 + jl;
                if (j >= len) vr[u] = *reinterpret_cast<const float4*>(nv + (j - len) * D + 4 * c4);
#pragma unroll
                for (int qi = 0; qi < QB; ++qi) {
                    if (qi >= Q) break;
                    const float p = sp[qi * C + jl];
                    o[qi].x = fmaf(p, vr[u].x, o[qi].x);
                    o[qi].y = fmaf(p, vr[u].y, o[qi].y);
                    o[qi].z = fmaf(p, vr[u].z, o[qi].z);
                    o[qi].w = fmaf(p, vr[u].w, o[qi].w);
                }
            }
        };
        for (int it = 0; it < nit_v; it += 2) {
            if (it > 0 && it + 1 < nit_v) load_v(vB, it + 1);
            accumulate(vA, it);
            if (it + 1 < nit_v) {
                if (it + 2 < nit_v) load_v(vA, it + 2);
                accumulate(vB, it + 1);
            }
        }
        // the NG groups' sums: the groups of one wave by lane shuffles, then the
        // four waves through red[w][qi][D], added up when the triples are written
        constexpr int GPW = 64 / D4;  // groups per wave (4, 2, 1)
#pragma unroll
        for (int qi = 0; qi < QB; ++qi) {
            if (qi >= Q) continue;  // wave-uniform
            float4 v = o[qi];
            if constexpr (GPW >= 4) {
                v.x += __shfl_xor(v.x, 16, 64); v.y += __shfl_xor(v.y, 16, 64);
                v.z += __shfl_xor(v.z, 16, 64); v.w += __shfl_xor(v.w, 16, 64);
            }
            if constexpr (GPW >= 2) {
                v.x += __shfl_xor(v.x, 32, 64); v.y += __shfl_xor(v.y, 32, 64);
                v.z += __shfl_xor(v.z, 32, 64); v.w += __shfl_xor(v.w, 32, 64);
            }
            if (lane < D4) *reinterpret_cast<float4*>(red + (wv * QB + qi) * D + 4 * c4) = v;
        }
    }
    __syncthreads();

    // 6. the chunk's (max, sum) pair and o of every query (ms [q][chunk][2], po
    //    [q][chunk][D], q = t H + h)
    float* ms = part;
    float* po = part + (int64_t)m * H * chunks * 2;
    for (int i = tid; i < Q * D; i += kThreads) {
        const int qi = i / D, d = i - qi * D;
        const int t = qi / G, e = qi - t * G;
        const int64_t qc = ((int64_t)t * H + g * G + e) * chunks + c;
        if (d == 0) *reinterpret_cast<float2*>(ms + 2 * qc) = make_float2(stat[2 * qi], stat[2 * qi + 1]);
        po[qc * D + d] = (red[qi * D + d] + red[(QB + qi) * D + d]) +
                         (red[(2 * QB + qi) * D + d] + red[(3 * QB + qi) * D + d]);
    }
}

// The merge, per (token t, head h) = blockIdx.x: wave 0 reads every chunk's (max, sum)
// pair (one pass of loads), forms the overall max M and sum S and each chunk's weight
// e^(M_c - M) / S in LDS; thread d sums o_c[d] times the weights, 32 chunks' loads in
// flight (the first 32 requested at entry).  A chunk whose queries were all masked has M_c = -inf and weight 0.
// The cache length advances here (workgroup 0, after every chunk has read it), or,
// when the call found len + m > max_seq, the output is NaN and the overflow flag set.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(const float* __restrict__ part, int m,
                                                       int H, int chunks, float* __restrict__ out,
                                                       int* __restrict__ state, int max_seq) {
    extern __shared__ float wts[];  // [chunks] weights, then [chunks] the chunks' sums
    const int th = blockIdx.x;      // t H + h
    const int tid = threadIdx.x, lane = tid & 63;
    const float2* pq = reinterpret_cast<const float2*>(part) + (int64_t)th * chunks;
    const float* po = part + (int64_t)m * H * chunks * 2 + (int64_t)th * chunks * D + tid;
    // every load that needs no other is requested at once, before the length is
    // checked: the length, the first 64 chunks' (max, sum) and the first 32 chunks'
    // o[d] (the o loads do not depend on the weights, so they overlap the (max, sum)
    // pass)
    const int len = state[2];
    float2 v0 = make_float2(-INFINITY, 0.0f);
    if (tid < 64 && lane < chunks) v0 = pq[lane];
    float ov[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) ov[u] = po[(int64_t)min(u, chunks - 1) * D];
    if (len + m > max_seq) {
        out[(int64_t)th * D + tid] = __builtin_nanf("");
        if (th == 0 && tid == 0) state[1] = 1;
        return;
    }
    if (th == 0 && tid == 0) state[0] = len + m;
    if (tid < 64) {
        float* sy = wts + chunks;
        float M = v0.x;
        if (lane < chunks) {
            wts[lane] = v0.x;
            sy[lane] = v0.y;
        }
        for (int cc = lane + 64; cc < chunks; cc += 64) {
            const float2 v = pq[cc];
            wts[cc] = v.x;
            sy[cc] = v.y;
            M = fmaxf(M, v.x);
        }
        M = wave_max(M);
        float S = 0.0f;
        for (int cc = lane; cc < chunks; cc += 64) {
            const float mc = wts[cc];
            const float f = M == -INFINITY || mc == -INFINITY ? 0.0f : expf(mc - M);
            wts[cc] = f;
            S = fmaf(sy[cc], f, S);
        }
        S = wave_add(S);
        for (int cc = lane; cc < chunks; cc += 64) wts[cc] /= S;
    }
    __syncthreads();
    float O = 0.0f;
    for (int cc = 0; cc < chunks; cc += 32) {  // the last batch clamps its loads
        if (cc > 0)
#pragma unroll
            for (int u = 0; u < 32; ++u) ov[u] = po[(int64_t)min(cc + u, chunks - 1) * D];
#pragma unroll
        for (int u = 0; u < 32; ++u)
            if (cc + u < chunks) O = fmaf(ov[u], wts[cc + u], O);
    }
    out[(int64_t)th * D + tid] = O;
}

template <int D, int QB>
hipError_t launch_d_q(const KvCache& kv, const float* qkv, int m, int H, int C, int chunks,
                      float* part, float* out, hipStream_t s) {
    const size_t lds = sizeof(float) * ((size_t)QB * D * 5 + (size_t)m * D * 2 +
                                        (size_t)QB * C + 2 * QB);
    if (lds > 159 * 1024) return hipErrorInvalidValue;
    static const bool attr = hipFuncSetAttribute((const void*)attn_decode_kernel<D, QB>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 160 * 1024 - 1024) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    attn_decode_kernel<D, QB><<<dim3((unsigned)kv.n_kv_heads, (unsigned)chunks), kThreads, lds, s>>>(
        qkv, m, H, (int)kv.n_kv_heads, kv.state, C, chunks, 1.0f / sqrtf((float)D), kv.inv_freq,
        kv.k, kv.v, (int)kv.max_seq, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_merge_kernel<D><<<(unsigned)(m * H), D, sizeof(float) * 2 * (size_t)chunks, s>>>(
        part, m, H, chunks, out, kv.state, (int)kv.max_seq);
    return hipGetLastError();
}

template <int D>
hipError_t launch_d(const KvCache& kv, const float* qkv, int m, int H, int C, int chunks,
                    float* part, float* out, hipStream_t s) {
    const int Q = m * (H / (int)kv.n_kv_heads);
    if (Q <= 1) return launch_d_q<D, 1>(kv, qkv, m, H, C, chunks, part, out, s);
    if (Q <= 2) return launch_d_q<D, 2>(kv, qkv, m, H, C, chunks, part, out, s);
    if (Q <= 4) return launch_d_q<D, 4>(kv, qkv, m, H, C, chunks, part, out, s);
    if (Q <= 8) return launch_d_q<D, 8>(kv, qkv, m, H, C, chunks, part, out, s);
    return launch_d_q<D, 16>(kv, qkv, m, H, C, chunks, part, out, s);
}

// Chunk length for L positions: (kv head, chunk) workgroups to cover the CUs
// twice; chunks of 32 .. kMaxChunk positions (a multiple of 32), at most
// kMaxChunks of them.  0 when L is beyond kMaxChunk * kMaxChunks.
int64_t chunk_len(int64_t L, int64_t KVH) {
    // chunks for 4x the CUs up to 2048 positions, 2x beyond (MHA L1024: 12.7 -> 12.2 us
    // a call with 4x; L4096 measured slower with 4x, 31.2 against 27.1 us)
    const int64_t want = (L <= 2048 ? 4 : 2) * (int64_t)device_info().cu_count;
    // enough chunks for the CUs, but none longer than kMaxChunk: with many kv heads
    // the CUs fill with fewer, longer chunks, and the cap takes over from there
    int64_t C = std::min<int64_t>((L * KVH + want - 1) / want, kMaxChunk);
    C = std::max(C, (L + kMaxChunks - 1) / kMaxChunks);
    C = std::max<int64_t>(32, (C + 31) / 32 * 32);
    return C > kMaxChunk ? 0 : C;
}

// ---- prompt-length calls (m H / KVH beyond a decode step) ---------------------------------
//
// rope_append_kernel, a workgroup per (token t, head): q heads rotated at position
// len + t and scaled by 1 / sqrt(hd) into the workspace qw[H][m][hd]; k heads rotated
// and, with v, appended to the cache (the decode kernel's formulas, so either path
// writes the same cache).  Then, for hd 64 and 128, attn_prefill_mfma on the f32 matrix
// cores (further down; with its key range split, attn_merge_split_kernel after it);
// for hd 256, attn_prefill_kernel, a workgroup per (block of BQ queries, head h):
// flash-style causal attention over the cache in f32 --
//   - the block's queries Q^T [hd][BQ] stay in LDS; the key positions run in tiles of BK
//     (K^T [hd][BK] and V [BK][hd] in LDS), only up to the block's last query position;
//   - thread (tr, tc) of 16 x 16 computes scores for rows tr RT .. and columns tc CT ..
//     (RT = BQ / 16, CT = BK / 16), masks positions past each query (and past the
//     filled length), and keeps each row's running max and sum (online softmax: the
//     earlier partial output rescaled by e^(m_old - m_new)); the row reductions run over
//     the 16 lanes of one tc group by lane shuffles;
//   - the exponentials go to LDS as P^T [BK][BQ]; the same thread then accumulates
//     rows tr RT .. of O for output dimensions tc hd / 16 .., read P and V from LDS.
// f32 throughout, like the reference's cache and matmuls (llama.rs:1108-1146).  LDS
// rows are padded by 4 floats so the transposing stores spread over the banks.

template <int D>
__global__ __launch_bounds__(D / 2) void rope_append_kernel(
    const float* __restrict__ qkv, int m, int H, int KVH, int* __restrict__ state, float scale,
    const float* __restrict__ inv_freq, float* __restrict__ kc, float* __restrict__ vc,
    int max_seq, float* __restrict__ qw) {
    constexpr int HALF = D / 2;
    const int len = state[0];
    const int t = blockIdx.x, hh = blockIdx.y, p = threadIdx.x;
    if (t == 0 && hh == 0 && p == 0) state[2] = len;  // this call's length, for the next kernel
    if (len + m > max_seq) return;  // overflow: nothing appended; the attention kernel reports it
    const float* row = qkv + (int64_t)t * (H + 2 * KVH) * D;
    float sn, cs;
    sincosf((float)(len + t) * inv_freq[p], &sn, &cs);
    if (hh < H) {
        const float* x = row + (int64_t)hh * D;
        const float a = x[p], b = x[p + HALF];
        float* q = qw + ((int64_t)hh * m + t) * D;
        q[p] = (a * cs - b * sn) * scale;
        q[p + HALF] = (a * sn + b * cs) * scale;
    } else {
        const int g = hh - H;
        const float* xk = row + (int64_t)(H + g) * D;
        const float* xv = row + (int64_t)(H + KVH + g) * D;
        const float a = xk[p], b = xk[p + HALF];
        const int64_t dst = ((int64_t)g * max_seq + len + t) * D;
        kc[dst + p] = a * cs - b * sn;
        kc[dst + p + HALF] = a * sn + b * cs;
        vc[dst + p] = xv[p];
        vc[dst + p + HALF] = xv[p + HALF];
    }
}

template <int D, int BQ, int BK>
struct PrefillLds {
    static constexpr int QP = BQ + 4, KP = BK + 4, VP = D + 4, PP = BQ + 4;  // padded rows
    static constexpr int FLOATS = D * QP + D * KP + BK * VP + BK * PP;
    static constexpr size_t BYTES = (size_t)FLOATS * sizeof(float);
};

template <int D, int BQ, int BK>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float* __restrict__ qw, int m,
                                                           int H, int KVH,
                                                           int* __restrict__ state,
                                                           const float* __restrict__ kc,
                                                           const float* __restrict__ vc,
                                                           int max_seq, float* __restrict__ out) {
    using L = PrefillLds<D, BQ, BK>;
    constexpr int RT = BQ / 16, CT = BK / 16, DC = D / 16;
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* qT = sm;                 // [D][QP]
    float* kT = qT + D * L::QP;     // [D][KP]
    float* vs = kT + D * L::KP;     // [BK][VP]
    float* pT = vs + BK * L::VP;    // [BK][PP]
    const int h = blockIdx.y, g = h / (H / KVH);
    const int q0 = blockIdx.x * BQ;
    const int tid = threadIdx.x, tr = tid / 16, tc = tid % 16;
    const int len = state[2];
    const int nq = min(BQ, m - q0);  // real queries of the block
    if (len + m > max_seq) {
        for (int i = tid; i < nq * D; i += 256)
            out[(int64_t)(q0 + i / D) * H * D + (int64_t)h * D + i % D] = __builtin_nanf("");
        if (blockIdx.x == 0 && h == 0 && tid == 0) state[1] = 1;
        return;
    }
    // the length advances here: no workgroup of this kernel reads state[0], and the next
    // call's kernels run after this one
    if (blockIdx.x == 0 && h == 0 && tid == 0) state[0] = len + m;
    const int total = len + m;  // filled positions once this call's keys are in
    // the block's queries, transposed (rows past m repeat the last query)
    for (int i = tid; i < BQ * D; i += 256) {
        const int r = i / D, d = i - r * D;
        qT[d * L::QP + r] = qw[((int64_t)h * m + min(q0 + r, m - 1)) * D + d];
    }
    float mrow[RT], lrow[RT], o[RT][DC];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        mrow[r] = -INFINITY;
        lrow[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < DC; ++c) o[r][c] = 0.0f;
    }
    const int last_pos = len + q0 + nq - 1;  // the block's last query position
    const int nkb = last_pos / BK + 1;
    const float* kg = kc + (int64_t)g * max_seq * D;
    const float* vg = vc + (int64_t)g * max_seq * D;
    for (int kb = 0; kb < nkb; ++kb) {
        __syncthreads();  // the previous tile's readers are done (and Q is staged)
        for (int i = tid; i < BK * D; i += 256) {
            const int j = i / D, d = i - j * D;
            const int64_t src = (int64_t)min(kb * BK + j, total - 1) * D + d;
            kT[d * L::KP + j] = kg[src];
            vs[j * L::VP + d] = vg[src];
        }
        __syncthreads();
        float s[RT][CT];
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int c = 0; c < CT; ++c) s[r][c] = 0.0f;
        for (int d = 0; d < D; ++d) {
            float qv[RT], kv[CT];
#pragma unroll
            for (int r = 0; r < RT; ++r) qv[r] = qT[d * L::QP + tr * RT + r];
#pragma unroll
            for (int c = 0; c < CT; ++c) kv[c] = kT[d * L::KP + tc * CT + c];
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < CT; ++c) s[r][c] = fmaf(qv[r], kv[c], s[r][c]);
        }
        // causal mask (position j visible to query i when j <= len + i), running max
        // and sum per row over the 16 lanes of the row group
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const int qpos = len + q0 + tr * RT + r;
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const int kpos = kb * BK + tc * CT + c;
                if (kpos > qpos || kpos >= total) s[r][c] = -INFINITY;
                mx = fmaxf(mx, s[r][c]);
            }
#pragma unroll
            for (int o2 = 8; o2 > 0; o2 >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o2, 16));
            const float mnew = fmaxf(mrow[r], mx);
            const float alpha = mnew == -INFINITY ? 1.0f : expf(mrow[r] - mnew);
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const float p = s[r][c] == -INFINITY ? 0.0f : expf(s[r][c] - mnew);
                s[r][c] = p;
                sum += p;
            }
#pragma unroll
            for (int o2 = 8; o2 > 0; o2 >>= 1) sum += __shfl_xor(sum, o2, 16);
            lrow[r] = lrow[r] * alpha + sum;
            mrow[r] = mnew;
#pragma unroll
            for (int c = 0; c < DC; ++c) o[r][c] *= alpha;
#pragma unroll
            for (int c = 0; c < CT; ++c) pT[(tc * CT + c) * L::PP + tr * RT + r] = s[r][c];
        }
        __syncthreads();
        for (int j = 0; j < BK; ++j) {
            float pv[RT], vv[DC];
#pragma unroll
            for (int r = 0; r < RT; ++r) pv[r] = pT[j * L::PP + tr * RT + r];
#pragma unroll
            for (int c = 0; c < DC; ++c) vv[c] = vs[j * L::VP + tc * DC + c];
#pragma unroll
            for (int r = 0; r < RT; ++r)
#pragma unroll
                for (int c = 0; c < DC; ++c) o[r][c] = fmaf(pv[r], vv[c], o[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const int qi = q0 + tr * RT + r;
        if (qi >= m) continue;
        const float inv = 1.0f / lrow[r];
#pragma unroll
        for (int c = 0; c < DC; ++c)
            out[(int64_t)qi * H * D + (int64_t)h * D + tc * DC + c] = o[r][c] * inv;
    }
}

// ---- prompt-length attention on the f32 matrix cores (hd 64 and 128) ------------------------
//
// attn_prefill_mfma<D, NW>: a workgroup per (NW / 2 pairs of 32-query tiles, head h), NW
// waves, each owning one tile (the pairing below balances the causal work).  Everything is f32: v_mfma_f32_32x32x2f32
// multiplies f32 operands exactly and accumulates in f32, like the FMA loop above, so
// the numbers match it to summation order.  The products are formed transposed so that
// no row reduction crosses more than two lanes and P never leaves the registers:
//   S^T [32 keys][32 queries] = K . Q^T -- the MFMA's A operand is a key row (lane l:
//     key l % 32), B is the wave's queries (lane l: query l % 32), and MFMA s contracts
//     dimensions s and D / 2 + s (lane half l / 32 takes one of each pair), so a lane
//     reads its key's dimensions as float4s from LDS and keeps its query's half in
//     registers for the whole kernel;
//   a lane's 16 accumulators are 16 keys of ONE query (rows 8 (r / 4) + 4 (l / 32) +
//     r % 4, column l % 32): the query's max and sum over the tile are a 16-value
//     register reduction and one exchange with lane l ^ 32;
//   O^T [D][32 queries] += V^T . P^T -- MFMA s contracts keys 8 (s / 4) + s % 4 and the
//     same + 4, exactly the two keys whose exponentials lanes l and l ^ 32 hold in
//     accumulator s: B is the lane's own p[s], A is V[that key][32 t + l % 32] (D / 32
//     output tiles).
// Key tiles of 32 positions (K and V rows padded to D + 4 floats in LDS) are double
// buffered: tile k + 1 is read into registers while tile k is computed and stored to
// LDS after it.  A wave skips the tiles wholly past its last query (causal) but keeps
// loading and meeting the others.  Same length and overflow handling as
// attn_prefill_kernel.
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int D, int NW>
struct MfmaPrefillLds {
    static constexpr int ROW = D + 4;                     // padded row (floats)
    static constexpr int TILE = 32 * ROW;                 // one of K or V, or a wave's queries
    static constexpr size_t BYTES = (size_t)2 * 2 * TILE * sizeof(float);  // 2 stages x (K, V)
    static constexpr int LPT = 2 * 32 * D / 4 / (64 * NW);  // float4 loads a thread per tile
};

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void attn_prefill_mfma(const float* __restrict__ qw, int m,
                                                             int H, int KVH,
                                                             int* __restrict__ state,
                                                             const float* __restrict__ kc,
                                                             const float* __restrict__ vc,
                                                             int max_seq, float* __restrict__ out,
                                                             float* __restrict__ part) {
    using L = MfmaPrefillLds<D, NW>;
    constexpr int HALF = D / 2, OT = D / 32, ROW = L::ROW;
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int h = blockIdx.y, g = h / (H / KVH);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int col = lane & 31, hf = lane >> 5;
    // The head's T tiles of 32 queries are paired (i, T - 1 - i), so that under the
    // causal mask every pair holds the same work (the middle tile of an odd T has no
    // partner); workgroup b takes pairs b NW / 2 .. + NW / 2 - 1, waves w < NW / 2
    // their low tiles and the others their high ones (one of each a SIMD).  -1: no
    // tile for this wave.
    const int T = (m + 31) / 32, P = (T + 1) / 2;
    auto tile_of = [&](int w) {
        const int i = (int)blockIdx.x * (NW / 2) + w % (NW / 2);
        if (i >= P) return -1;
        if (w < NW / 2) return i;
        return T - 1 - i > i ? T - 1 - i : -1;
    };
    const int mytile = tile_of(wv);  // wave-uniform
    int top = 0;                     // the workgroup's last tile
#pragma unroll
    for (int w = 0; w < NW; ++w) top = max(top, tile_of(w));
    // gridDim.z > 1: this workgroup takes split blockIdx.z of the key tiles and writes
    // partials (max, sum, unnormalized o) for attn_merge_kernel, which then also
    // advances the length or reports the overflow
    const int S = gridDim.z, z = blockIdx.z;
    const int len = state[2];
    if (len + m > max_seq) {
        if (S == 1) {
            if (mytile >= 0)
                for (int i = lane; i < 32 * D; i += 64) {
                    const int q = 32 * mytile + i / D;
                    if (q < m) out[(int64_t)q * H * D + (int64_t)h * D + i % D] = __builtin_nanf("");
                }
            if (blockIdx.x == 0 && h == 0 && tid == 0) state[1] = 1;
        }
        return;
    }
    if (S == 1 && blockIdx.x == 0 && h == 0 && tid == 0) state[0] = len + m;
    const int total = len + m;
    const float* kg = kc + (int64_t)g * max_seq * D;
    const float* vg = vc + (int64_t)g * max_seq * D;

    // this lane's query (rows past m, and a wave without a tile, repeat the last one),
    // its half of the dimensions in one vector (a vector stays in registers)
    const int qi = mytile >= 0 ? 32 * mytile + col : m;
    typedef float qhalf_t __attribute__((ext_vector_type(HALF)));
    qhalf_t qr;
    {
        const float* qrow = qw + ((int64_t)h * m + min(qi, m - 1)) * D + hf * HALF;
#pragma unroll
        for (int u = 0; u < HALF / 4; ++u) {
            const float4 v = *reinterpret_cast<const float4*>(qrow + 4 * u);
            qr[4 * u] = v.x;
            qr[4 * u + 1] = v.y;
            qr[4 * u + 2] = v.z;
            qr[4 * u + 3] = v.w;
        }
    }
    const int qpos = len + qi;  // this lane's query position
    // the wave's last query position (-1: no tile, every key tile skipped)
    const int wave_last = mytile >= 0 ? len + min(32 * mytile + 31, m - 1) : -1;
    const int last_pos = len + min(32 * top + 31, m - 1);
    const int ntiles = last_pos / 32 + 1;
    const int kt0 = z * ntiles / S, kt1 = (z + 1) * ntiles / S;  // this workgroup's key tiles

    // tile loads: float4 f = i (64 NW) + tid, i < LPT, over [K rows 0..31 | V rows 0..31];
    // the staged floats sit in one vector (a vector stays in registers)
    typedef float stage_t __attribute__((ext_vector_type(4 * L::LPT)));
    stage_t st;
    auto src_of = [&](int i, int kt) {
        const int f = i * 64 * NW + tid;
        const int which = f / (32 * D / 4), r = (f / (D / 4)) % 32, c = f % (D / 4);
        return (which ? vg : kg) + (int64_t)min(kt * 32 + r, total - 1) * D + 4 * c;
    };
    auto dst_of = [&](int i) {
        const int f = i * 64 * NW + tid;
        const int which = f / (32 * D / 4), r = (f / (D / 4)) % 32, c = f % (D / 4);
        return which * L::TILE + r * ROW + 4 * c;
    };

    float mrun = -INFINITY, lrun = 0.0f;
    f32x16 o[OT];
#pragma unroll
    for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t][e] = 0.0f;

#pragma unroll
    for (int i = 0; i < L::LPT; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(src_of(i, kt0));
        *reinterpret_cast<float4*>(sm + (kt0 & 1) * 2 * L::TILE + dst_of(i)) = v;
    }
    __syncthreads();
    for (int kt = kt0; kt < kt1; ++kt) {
        const float* Ks = sm + (kt & 1) * 2 * L::TILE;
        const float* Vs = Ks + L::TILE;
        const bool more = kt + 1 < kt1;
        const bool live = kt * 32 <= wave_last;  // wave-uniform: tiles past the wave's last query skipped
        f32x16 s;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = 0.0f;
        if (live) {
            // S^T = K . Q^T, the next float4 of the key row read ahead of the MFMAs
            const float* krow = Ks + col * ROW + hf * HALF;
            // two accumulators (dimension pairs alternate), so consecutive MFMAs do not
            // wait on each other's results
            f32x16 s2;
#pragma unroll
            for (int e = 0; e < 16; ++e) s2[e] = 0.0f;
            float4 kv = *reinterpret_cast<const float4*>(krow);
#pragma unroll
            for (int u = 0; u < HALF / 4; ++u) {
                const float4 kn =
                    u + 1 < HALF / 4 ? *reinterpret_cast<const float4*>(krow + 4 * (u + 1)) : kv;
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qr[4 * u], s, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qr[4 * u + 1], s2, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qr[4 * u + 2], s, 0, 0, 0);
                s2 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qr[4 * u + 3], s2, 0, 0, 0);
                kv = kn;
            }
            s += s2;
        }
        // the next tile's rows requested while this one's softmax and p v run
        if (more) {
#pragma unroll
            for (int i = 0; i < L::LPT; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(src_of(i, kt + 1));
                st[4 * i] = v.x;
                st[4 * i + 1] = v.y;
                st[4 * i + 2] = v.z;
                st[4 * i + 3] = v.w;
            }
        }
        if (live) {
            // causal mask and the query's running max / sum
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kpos = kt * 32 + 8 * (r / 4) + 4 * hf + r % 4;
                if (kpos > qpos || kpos >= total) s[r] = -INFINITY;
                tmax = fmaxf(tmax, s[r]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(mrun, tmax);
            const float alpha = mnew == -INFINITY ? 1.0f : expf(mrun - mnew);
            float tsum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = s[r] == -INFINITY ? 0.0f : expf(s[r] - mnew);
                s[r] = p;
                tsum += p;
            }
            tsum += __shfl_xor(tsum, 32, 64);
            lrun = lrun * alpha + tsum;
            mrun = mnew;
            // O^T = alpha O^T + V^T . P^T.  The rescale moves the accumulators through
            // the VALU, so it runs only when some query's running max changed (alpha
            // is then < 1 somewhere in the wave; after the first tiles it rarely is).
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int t = 0; t < OT; ++t)
#pragma unroll
                    for (int e = 0; e < 16; ++e) o[t][e] *= alpha;
            }
            // two output tiles at a time, their MFMAs interleaved (independent chains),
            // the tiles' 32 V values read ahead
#pragma unroll
            for (int t = 0; t < OT; t += 2) {
                float vv[2][16];
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        vv[a][r] = Vs[(8 * (r / 4) + 4 * hf + r % 4) * ROW + 32 * (t + a) + col];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[0][r], s[r], o[t], 0, 0, 0);
                    o[t + 1] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(vv[1][r], s[r], o[t + 1], 0, 0, 0);
                }
            }
        }
        if (more) {
            float* base = sm + ((kt + 1) & 1) * 2 * L::TILE;
#pragma unroll
            for (int i = 0; i < L::LPT; ++i)
                *reinterpret_cast<float4*>(base + dst_of(i)) =
                    make_float4(st[4 * i], st[4 * i + 1], st[4 * i + 2], st[4 * i + 3]);
        }
        __syncthreads();
    }
    if (S > 1) {
        // partials as attn_merge_kernel reads them: (max, sum) at [q H + h][S], o at
        // [q H + h][S][hd] after all the pairs (a query with no live tile in this split
        // leaves (-inf, 0) and zeros, weight 0 in the merge)
        if (qi < m) {
            const int64_t qc = ((int64_t)qi * H + h) * S + z;
            if (hf == 0) *reinterpret_cast<float2*>(part + 2 * qc) = make_float2(mrun, lrun);
            float* prow = part + (int64_t)m * H * S * 2 + qc * D + 4 * hf;
#pragma unroll
            for (int t = 0; t < OT; ++t)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    *reinterpret_cast<float4*>(prow + 32 * t + 8 * u) =
                        make_float4(o[t][4 * u], o[t][4 * u + 1], o[t][4 * u + 2], o[t][4 * u + 3]);
        }
        return;
    }
    // O[q][32 t + 8 u + 4 hf + 0..3] = o[t][4 u + 0..3] / l, a float4 each
    if (qi < m) {
        const float inv = 1.0f / lrun;
        float* orow = out + (int64_t)qi * H * D + (int64_t)h * D + 4 * hf;
#pragma unroll
        for (int t = 0; t < OT; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                *reinterpret_cast<float4*>(orow + 32 * t + 8 * u) =
                    make_float4(o[t][4 * u] * inv, o[t][4 * u + 1] * inv, o[t][4 * u + 2] * inv,
                                o[t][4 * u + 3] * inv);
    }
}

// The merge of a split prompt call (S splits of each workgroup's key tiles, a handful):
// a thread per (query q, head h, 4 dimensions); out = sum_z e^(M_z - M) o_z /
// sum_z e^(M_z - M) l_z over the splits' (M_z, l_z, o_z) partials (a split in which the
// query had no live key leaves M_z = -inf: weight 0).  The length advance and the
// overflow report are attn_merge_kernel's.
template <int D>
__global__ __launch_bounds__(256) void attn_merge_split_kernel(const float* __restrict__ part,
                                                               int m, int H, int S,
                                                               float* __restrict__ out,
                                                               int* __restrict__ state,
                                                               int max_seq) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (q H + h) (D / 4) + d4
    const int64_t total = (int64_t)m * H * (D / 4);
    const int len = state[2];
    if (len + m > max_seq) {
        if (i < total)
            reinterpret_cast<float4*>(out)[i] =
                make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                            __builtin_nanf(""));
        if (i == 0) state[1] = 1;
        return;
    }
    if (i == 0) state[0] = len + m;
    if (i >= total) return;
    const int64_t qh = i / (D / 4), d4 = i % (D / 4);
    const float2* ms = reinterpret_cast<const float2*>(part) + qh * S;
    const float4* po = reinterpret_cast<const float4*>(part + (int64_t)m * H * S * 2) + qh * S * (D / 4) + d4;
    float M = -INFINITY;
    for (int z = 0; z < S; ++z) M = fmaxf(M, ms[z].x);
    float l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < S; ++z) {
        const float2 p = ms[z];
        const float f = p.x == -INFINITY ? 0.0f : expf(p.x - M);
        const float4 v = po[(int64_t)z * (D / 4)];
        l = fmaf(p.y, f, l);
        o = make_float4(fmaf(v.x, f, o.x), fmaf(v.y, f, o.y), fmaf(v.z, f, o.z), fmaf(v.w, f, o.w));
    }
    const float inv = 1.0f / l;
    reinterpret_cast<float4*>(out)[i] = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

template <int D, int NW>
hipError_t launch_prefill_mfma(const KvCache& kv, const float* qkv, int m, int H, float* qw,
                               float* part, int S, float* out, hipStream_t s) {
    using L = MfmaPrefillLds<D, NW>;
    static const bool attr = hipFuncSetAttribute((const void*)attn_prefill_mfma<D, NW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)L::BYTES) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    const int KVH = (int)kv.n_kv_heads;
    rope_append_kernel<D><<<dim3((unsigned)m, (unsigned)(H + KVH)), D / 2, 0, s>>>(
        qkv, m, H, KVH, kv.state, 1.0f / sqrtf((float)D), kv.inv_freq, kv.k, kv.v,
        (int)kv.max_seq, qw);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // pairs of 32-query tiles, NW / 2 pairs a workgroup; S splits of the key tiles
    const int pairs = ((m + 31) / 32 + 1) / 2;
    attn_prefill_mfma<D, NW><<<dim3((unsigned)((pairs + NW / 2 - 1) / (NW / 2)), (unsigned)H,
                                    (unsigned)S),
                               64 * NW, L::BYTES, s>>>(qw, m, H, KVH, kv.state, kv.k, kv.v,
                                                       (int)kv.max_seq, out, part);
    e = hipGetLastError();
    if (S == 1 || e != hipSuccess) return e;
    const int64_t merge_threads = (int64_t)m * H * (D / 4);
    attn_merge_split_kernel<D><<<(unsigned)((merge_threads + 255) / 256), 256, 0, s>>>(
        part, m, H, S, out, kv.state, (int)kv.max_seq);
    return hipGetLastError();
}

// The largest workgroup (8, 4 or 2 waves of 32 queries) whose grid, with the call's S
// key splits, still gives every CU a workgroup: eight waves are two a SIMD (the K and V
// tiles in LDS allow only two workgroups a CU).
template <int D>
hipError_t launch_prefill_mfma_auto(const KvCache& kv, const float* qkv, int m, int H, float* qw,
                                    float* part, int S, float* out, hipStream_t s) {
    const int64_t cus = device_info().cu_count, pairs = ((m + 31) / 32 + 1) / 2;
    auto wgs = [&](int nw) { return (pairs + nw / 2 - 1) / (nw / 2) * H * S; };
    if (wgs(8) >= cus) return launch_prefill_mfma<D, 8>(kv, qkv, m, H, qw, part, S, out, s);
    if (wgs(4) >= cus) return launch_prefill_mfma<D, 4>(kv, qkv, m, H, qw, part, S, out, s);
    return launch_prefill_mfma<D, 2>(kv, qkv, m, H, qw, part, S, out, s);
}

template <int D, int BQ, int BK>
hipError_t launch_prefill_attn(const KvCache& kv, const float* qkv, int m, int H, float* qw,
                               float* out, hipStream_t s) {
    using L = PrefillLds<D, BQ, BK>;
    static const bool attr = hipFuncSetAttribute((const void*)attn_prefill_kernel<D, BQ, BK>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)L::BYTES) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    const int KVH = (int)kv.n_kv_heads;
    rope_append_kernel<D><<<dim3((unsigned)m, (unsigned)(H + KVH)), D / 2, 0, s>>>(
        qkv, m, H, KVH, kv.state, 1.0f / sqrtf((float)D), kv.inv_freq, kv.k, kv.v,
        (int)kv.max_seq, qw);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_prefill_kernel<D, BQ, BK><<<dim3((unsigned)((m + BQ - 1) / BQ), (unsigned)H), 256,
                                     L::BYTES, s>>>(qw, m, H, KVH, kv.state, kv.k, kv.v,
                                                    (int)kv.max_seq, out);
    return hipGetLastError();
}

}  // namespace

namespace {
// Key-range splits of a prompt call on the matrix-core kernel: the largest of 1, 2, 4
// that keeps the call's 32-query waves at most two a SIMD (m512 at 32 heads: 512
// waves on 1024 SIMDs, 4 splits); 1 needs no partials and no merge.
int prompt_split(int64_t m, int64_t H, int64_t D) {
    if (D != 64 && D != 128) return 1;
    const int64_t waves = (m + 31) / 32 * H, target = 8 * (int64_t)device_info().cu_count;
    int S = 1;
    while (S < 4 && waves * 2 * S <= target) S *= 2;
    return S;
}
size_t prompt_q_bytes(int64_t m, int64_t H, int64_t D) {
    return ((size_t)m * H * D * sizeof(float) + 255) / 256 * 256;
}
}  // namespace

namespace {
// Workspace (slot 2) of one call of m tokens: the decode path's per-chunk partials at
// any length (at most kMaxChunks chunks of (max, sum) and o[hd] per query), or the
// prompt path's rotated queries [H][m][hd] followed, for a split call, by its S
// partials per query.
size_t attention_call_bytes(const KvCache& kv, int64_t m, int64_t H) {
    const int64_t G = H / std::max<int64_t>(kv.n_kv_heads, 1), D = kv.head_dim;
    if (m * G <= kAttnMaxQ) return (size_t)m * H * kMaxChunks * (2 + D) * sizeof(float);
    const int S = prompt_split(m, H, D);
    return prompt_q_bytes(m, H, D) + (S > 1 ? (size_t)m * H * S * (2 + D) * sizeof(float) : 0);
}
}  // namespace

// Enough for every call of up to m tokens (what unillm_hip_attention_reserve grows to).
// A call's need grows with m inside each regime -- decode, then prompts with 4, 2 and
// 1 key splits -- but not across them (a split 512-token prompt takes more than an
// unsplit 2048-token one), so the largest lies at the right end of a regime, clipped
// to m.
size_t attention_workspace_bytes(const KvCache& kv, int64_t m, int64_t H) {
    const int64_t G = H / std::max<int64_t>(kv.n_kv_heads, 1);
    const int64_t target = 8 * (int64_t)device_info().cu_count;  // prompt_split's two a SIMD
    const int64_t ends[4] = {m, kAttnMaxQ / G, 32 * (target / (4 * H)), 32 * (target / (2 * H))};
    size_t need = 0;
    for (int64_t c : ends) {
        c = std::min(c, m);
        if (c >= 1) need = std::max(need, attention_call_bytes(kv, c, H));
    }
    return need;
}

hipError_t launch_attention(const KvCache& kv, const float* qkv, int64_t m, int64_t H,
                            float* out, int64_t len_hint, hipStream_t s) {
    const int D = (int)kv.head_dim;
    void* ws = nullptr;
    hipError_t e;
    if (m * (H / kv.n_kv_heads) > kAttnMaxQ) {
        if ((e = stream_workspace(s, attention_call_bytes(kv, m, H), &ws, 2)) != hipSuccess)
            return e;
        float* qw = static_cast<float*>(ws);
        float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + prompt_q_bytes(m, H, D));
        const int S = prompt_split(m, H, D);
        if (D == 64)
            return launch_prefill_mfma_auto<64>(kv, qkv, (int)m, (int)H, qw, part, S, out, s);
        if (D == 128)
            return launch_prefill_mfma_auto<128>(kv, qkv, (int)m, (int)H, qw, part, S, out, s);
        return launch_prefill_attn<256, 32, 32>(kv, qkv, (int)m, (int)H, qw, out, s);
    }
    // decode: chunks sized for the known length, or for the longest the cache holds
    const int64_t L = len_hint >= 0 ? len_hint + m
                                    : std::min<int64_t>(kv.max_seq, attention_max_positions());
    const int64_t C = chunk_len(L, kv.n_kv_heads);
    if (C == 0) return hipErrorInvalidValue;  // longer than kMaxChunk * kMaxChunks
    const int chunks = (int)((L + C - 1) / C);
    const size_t pbytes = (size_t)m * H * chunks * (2 + D) * sizeof(float);
    if ((e = stream_workspace(s, pbytes, &ws, 2)) != hipSuccess) return e;
    float* part = static_cast<float*>(ws);
    if (D == 64) return launch_d<64>(kv, qkv, (int)m, (int)H, (int)C, chunks, part, out, s);
    if (D == 128) return launch_d<128>(kv, qkv, (int)m, (int)H, (int)C, chunks, part, out, s);
    return launch_d<256>(kv, qkv, (int)m, (int)H, (int)C, chunks, part, out, s);
}

int attention_max_queries() { return kAttnMaxQ; }
int64_t attention_max_positions() { return (int64_t)kMaxChunk * kMaxChunks; }

}  // namespace unillm
