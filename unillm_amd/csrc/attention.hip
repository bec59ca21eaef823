// attention.hip -- decode attention with a KV cache in HBM (m new tokens, m <= 16).
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
// Three kernels on the caller's stream:
//   1. rope_append_kernel: one wave per (token, head) of the fused QKV row:
//      q heads rotated into the workspace, k heads rotated into the cache, v
//      heads copied into it.
//   2. attn_chunk_kernel: a workgroup per (kv head, chunk of C positions); its
//      four waves split the chunk, each lane holding hd / 64 dimensions of a
//      position's k and v, and run an online softmax for every query that
//      reads this kv head (the m tokens times the H / KVH heads of the group),
//      so each cached k and v is read from HBM once per step.  The waves'
//      (max, sum, weighted v) meet in LDS; the chunk's triple goes to the
//      workspace.
//   3. attn_merge_kernel: per (token, head), the chunks' triples merged by
//      log-sum-exp into the output row [m, H hd].
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <type_traits>

#include "internal.hpp"

namespace unillm {
namespace {

constexpr int kAttnMaxQ = 16;  // queries per kv head in one call: m * H / KVH

// rotation of the pair (x[i], x[i + hd / 2]) by pos * inv_freq[i]; lanes past hd / 2 idle
__global__ __launch_bounds__(128) void rope_append_kernel(const float* __restrict__ qkv, int H,
                                                          int KVH, int D,
                                                          const float* __restrict__ inv_freq,
                                                          int len, float* __restrict__ q_out,
                                                          float* __restrict__ kc,
                                                          float* __restrict__ vc, int max_seq) {
    const int t = blockIdx.x, h = blockIdx.y;  // token, head of the row (q, then k, then v)
    const int half = D / 2;
    const float* x = qkv + (int64_t)t * (H + 2 * KVH) * D + (int64_t)h * D;
    const int pos = len + t;
    if (h >= H + KVH) {  // v: copied
        float* dst = vc + ((int64_t)(h - H - KVH) * max_seq + pos) * D;
        for (int i = threadIdx.x; i < D; i += blockDim.x) dst[i] = x[i];
        return;
    }
    float* dst = h < H ? q_out + ((int64_t)t * H + h) * D
                       : kc + ((int64_t)(h - H) * max_seq + pos) * D;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float ang = (float)pos * inv_freq[i];
        float sn, cs;
        sincosf(ang, &sn, &cs);
        const float a = x[i], b = x[i + half];
        dst[i] = a * cs - b * sn;
        dst[i + half] = a * sn + b * cs;
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows(float v) {  // rows outside ROW_MASK read 0
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                         0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes, all in DPP (no LDS): each 16-lane row sums itself, then
// row_bcast:15 adds row 0 into row 1 and row 2 into row 3, row_bcast:31 rows 0-1
// into rows 2-3; lane 63 holds the total, read into a scalar for every lane.
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);  // row_ror:4
    v += dpp<0x128>(v);  // row_ror:8 -> every lane holds its row's sum
    v += dpp_rows<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_rows<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Workgroup (g, c): kv head g, positions [c C, min((c + 1) C, L)).  Queries of
// kv head g: token t, head h = g G + e (e < G) -> query qi = t G + e (Q = m G <=
// QB), whose causal limit is position len + t.  DPL = hd / 64 dimensions per
// lane; each wave takes U consecutive positions at a time (all their k and v
// requested before any is used), the four waves interleaved by U.
template <int DPL, int QB>
__global__ __launch_bounds__(256) void attn_chunk_kernel(const float* __restrict__ q, int m, int H,
                                                         int KVH, int len, int C, int chunks,
                                                         float scale, const float* __restrict__ kc,
                                                         const float* __restrict__ vc, int max_seq,
                                                         float* __restrict__ part) {
    constexpr int D = 64 * DPL, U = 8;
    const int g = blockIdx.x, c = blockIdx.y;
    const int G = H / KVH, Q = m * G;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int L = len + m;
    const int j0 = c * C, j1 = min(j0 + C, L);
    __shared__ float wred[4][QB][2];
    __shared__ float wo[4][QB * D];
    float qv[QB][DPL];  // this lane's dims of every query, pre-scaled by 1 / sqrt(hd)
#pragma unroll
    for (int qi = 0; qi < QB; ++qi)
#pragma unroll
        for (int d = 0; d < DPL; ++d) {
            const int t = min(qi, Q - 1) / G, e = min(qi, Q - 1) % G;
            qv[qi][d] = q[((int64_t)t * H + g * G + e) * D + d * 64 + lane] * scale;
        }
    float mx[QB], sm[QB], o[QB][DPL];
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) {
        mx[qi] = -INFINITY;
        sm[qi] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[qi][d] = 0.0f;
    }
    const float* kg = kc + (int64_t)g * max_seq * D;
    const float* vg = vc + (int64_t)g * max_seq * D;
    for (int jb = j0 + U * wv; jb < j1; jb += 4 * U) {
        float kj[U][DPL], vj[U][DPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = min(jb + u, j1 - 1);  // past the chunk: a repeat, skipped below
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                kj[u][d] = kg[j * D + d * 64 + lane];
                vj[u][d] = vg[j * D + d * 64 + lane];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = jb + u;
            if (j >= j1) break;  // wave-uniform
#pragma unroll
            for (int qi = 0; qi < QB; ++qi) {
                if (qi >= Q || j > len + qi / G) continue;  // causal (wave-uniform)
                float sv = 0.0f;
#pragma unroll
                for (int d = 0; d < DPL; ++d) sv = fmaf(qv[qi][d], kj[u][d], sv);
                sv = wave_sum64(sv);
                const float mn = fmaxf(mx[qi], sv);
                const float a = expf(mx[qi] - mn), pw = expf(sv - mn);
                sm[qi] = fmaf(sm[qi], a, pw);
#pragma unroll
                for (int d = 0; d < DPL; ++d) o[qi][d] = fmaf(o[qi][d], a, pw * vj[u][d]);
                mx[qi] = mn;
            }
        }
    }
    // the four waves' triples -> one per query
#pragma unroll
    for (int qi = 0; qi < QB; ++qi) {
        if (lane == 0) {
            wred[wv][qi][0] = mx[qi];
            wred[wv][qi][1] = sm[qi];
        }
#pragma unroll
        for (int d = 0; d < DPL; ++d) wo[wv][qi * D + d * 64 + lane] = o[qi][d];
    }
    __syncthreads();
    const int P = 2 + D;  // floats per (query, chunk) triple: max, sum, o[D]
    for (int i = threadIdx.x; i < Q * D; i += blockDim.x) {
        const int qi = i / D, d = i % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wred[w][qi][0]);
        float S = 0.0f, O = 0.0f;
        if (M != -INFINITY)
            for (int w = 0; w < 4; ++w) {
                const float f = wred[w][qi][0] == -INFINITY ? 0.0f : expf(wred[w][qi][0] - M);
                S += wred[w][qi][1] * f;
                O += wo[w][qi * D + d] * f;
            }
        const int t = qi / G, e = qi % G;
        float* dst = part + (((int64_t)t * H + g * G + e) * chunks + c) * P;
        if (d == 0) {
            dst[0] = M;
            dst[1] = S;
        }
        dst[2 + d] = O;
    }
}

// out[t, h D + d] = sum_c o_c e^(M_c - M) / sum_c S_c e^(M_c - M), one workgroup per
// (token, head): the chunks' maxima and sums reduced once by the workgroup, then
// 256 / D thread groups take every (256 / D)-th chunk of each dimension's sum
// (independent loads, unrolled) and meet in LDS.
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o, 64);
        v = is_max ? fmaxf(v, w) : v + w;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) red[wv] = v;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ part, int m,
                                                         int H, int D, int chunks,
                                                         float* __restrict__ out) {
    __shared__ float red[4];
    __shared__ float acc[256];
    const int th = blockIdx.x;  // token t * H + head h
    const int P = 2 + D;
    const float* pr = part + (int64_t)th * chunks * P;
    float M = -INFINITY;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) M = fmaxf(M, pr[c * P]);
    M = block_reduce(M, true, red);
    float S = 0.0f;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x)
        if (pr[c * P] != -INFINITY) S += pr[c * P + 1] * expf(pr[c * P] - M);
    S = block_reduce(S, false, red);
    const int groups = (int)blockDim.x / D;  // 4 (hd 64), 2 (128) or 1 (256)
    const int d = threadIdx.x % D, grp = threadIdx.x / D;
    float O = 0.0f;
#pragma unroll 8
    for (int c = grp; c < chunks; c += groups) {
        const float mc = pr[c * P];
        O += mc == -INFINITY ? 0.0f : pr[c * P + 2 + d] * expf(mc - M);
    }
    acc[threadIdx.x] = O;
    __syncthreads();
    if (grp == 0) {
        for (int gi = 1; gi < groups; ++gi) O += acc[gi * D + d];
        out[(int64_t)th * D + d] = O / S;
    }
}

}  // namespace

hipError_t launch_attention_decode(const KvCache& kv, const float* qkv, int64_t m, int64_t H,
                                   float* out, hipStream_t s) {
    const int D = (int)kv.head_dim, KVH = (int)kv.n_kv_heads, len = (int)kv.len;
    const int L = len + (int)m;
    // chunk length: enough (kv head, chunk) workgroups to cover the CUs twice
    const int64_t want = 2 * (int64_t)device_info().cu_count;
    int C = (int)std::max<int64_t>(32, ((int64_t)L * KVH + want - 1) / want);
    C = (C + 31) / 32 * 32;
    const int chunks = (L + C - 1) / C;
    const size_t qbytes = (size_t)m * H * D * sizeof(float);
    const size_t pbytes = (size_t)m * H * chunks * (2 + D) * sizeof(float);
    void* ws = nullptr;
    hipError_t e = stream_workspace(s, qbytes + pbytes, &ws, 2);
    if (e != hipSuccess) return e;
    float* qrot = static_cast<float*>(ws);
    float* part = qrot + (size_t)m * H * D;
    rope_append_kernel<<<dim3((unsigned)m, (unsigned)(H + 2 * KVH)), 128, 0, s>>>(
        qkv, (int)H, KVH, D, kv.inv_freq, len, qrot, kv.k, kv.v, (int)kv.max_seq);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const float scale = 1.0f / sqrtf((float)D);
    const dim3 grid((unsigned)KVH, (unsigned)chunks);
    const int Q = (int)(m * (H / KVH));
    auto go = [&](auto dpl, auto qb) {
        attn_chunk_kernel<decltype(dpl)::value, decltype(qb)::value><<<grid, 256, 0, s>>>(
            qrot, (int)m, (int)H, KVH, len, C, chunks, scale, kv.k, kv.v, (int)kv.max_seq, part);
    };
    auto by_q = [&](auto dpl) {
        using I = std::integral_constant<int, 1>;
        if (Q <= 1) go(dpl, I{});
        else if (Q <= 2) go(dpl, std::integral_constant<int, 2>{});
        else if (Q <= 4) go(dpl, std::integral_constant<int, 4>{});
        else if (Q <= 8) go(dpl, std::integral_constant<int, 8>{});
        else go(dpl, std::integral_constant<int, 16>{});
    };
    if (D == 64) by_q(std::integral_constant<int, 1>{});
    else if (D == 128) by_q(std::integral_constant<int, 2>{});
    else by_q(std::integral_constant<int, 4>{});
    if ((e = hipGetLastError()) != hipSuccess) return e;
    attn_merge_kernel<<<(unsigned)(m * H), 256, 0, s>>>(part, (int)m, (int)H, D, chunks, out);
    return hipGetLastError();
}

int attention_max_queries() { return kAttnMaxQ; }

}  // namespace unillm
