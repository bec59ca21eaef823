// prefill.hip -- fused dequant + f16 MFMA GEMM for prefill (m >= 65).
//
// y[m, n] = x[m, k] . dequant(W)[n, k]^T, the prefill call of QMatMul::forward
// (crates/runtime/src/models_v2/llama.rs:1188, 1329), fp32 accumulation on the
// gfx950 matrix cores.  Bound: MFMA (2 m n k flops over ~n k / 32 * 18 + 4 m k +
// 4 m n bytes).
// Operands are f16 (v_mfma_f32_16x16x32_f16).  Each row of x is scaled by a
// power of two that puts its largest magnitude in [2^14, 2^15) and rounded to
// f16 (xrows_kernel, or the fused layer norm); each weight is built from its
// code with the f16 magic number and rounded once, scaled by 2^-E (E: the
// weight's exponent offset).  Both scalings are exact and are undone on the
// output, so any finite x works, x and 2 x give the same operands, and the
// operands keep 11 significant bits.  ~1.75 VALU a weight (dequant8_f16),
// against ~3.25 for an fp32 dequant rounded to bf16 (this kernel's earlier
// form): 2-8 % faster per call, measured on one box.
//
// x is converted once, into the stream's workspace: the GEMM re-reads x once
// per 256-column tile, so half the bytes, and no conversion sits in its inner
// loop.
//
// Tile per workgroup: BM rows of x (BM = 256 or 128) x 256 weight rows
// (output columns), k in steps of 64 (two blocks).  Eight waves (two per
// SIMD) side by side: wave w owns all BM rows x columns 32 w .. 32 w + 31,
// BM / 16 x 2 MFMA tiles of 16 x 16, fp32 accumulators in registers.
//   - Operands reach LDS by direct global -> LDS loads through a 3- or 4-stage ring
//     (two k steps in flight, no VGPR staging): A as f16 rows with an XOR
//     swizzle of 16-byte chunks, B as the raw Q4_0 / Q8_0 payload bytes and
//     scales of the tile's 256 weight rows.
//   - Each lane reads the 8 payload bytes behind its MFMA B fragment and
//     dequantizes them in registers; every weight is dequantized once (a 2 x 4
//     grid of waves halves the A reads from LDS but dequantizes each column
//     twice: measured 10-30 % slower with the bf16 dequant, and still 5-10 %
//     slower with the f16 one, whose doubled cost matches the bf16 dequant done
//     once).
//   - The LDS reads are inline asm with explicit waits, so the compiler never
//     drains the ring's later stages before them; a step waits for its own
//     stage (vmcnt in issue order) and meets the other waves at a bare
//     s_barrier.
// Measured limits (m2048 k4096 n14336).  The loop alone -- these LDS reads, the MFMAs
// and a barrier a step, on operands already in LDS (a standalone probe, not built here)
// -- keeps the matrix cores 87-92 % busy.  Bringing each step's 42 KiB of operands
// from L2 into LDS costs about a quarter of the cycles however it is done (direct
// loads or through VGPRs, waited on or not): 68 %.  The dequant VALU does not overlap
// the same wave's MFMAs (copies of this kernel: without the dequant a call takes
// 86 % of the time, without the global loads 80 %, without both 75 %), and 448 tiles
// leave the last of two rounds a quarter idle.  A 2 x 4 wave grid halves the LDS
// reads but dequantizes every weight twice: 5-40 % slower.  MFMA accumulators in
// AGPRs, 7-wave tiles, s_setprio around the MFMAs, reads 3 or 4 ahead and the
// ring depth (3, 4 or 6 stages) made no difference.  Reading and dequantizing the
// next step's B during this step's MFMAs, so that a step starts straight into them,
// was 4-13 % slower (with the reads' wait deferred as well).  Dealing the tiles' k
// steps evenly over the CUs (1.75 tiles each at 448 tiles, split tiles summed from
// partial slots) gained nothing even with the cheapest slot exchange: with every
// CU busy each tile runs slower by about what the idle quarter round cost.
//
// Workgroup -> tile: workgroups are dealt round-robin over the 8 XCDs, so
// workgroup b takes tile (b % 8) * (T / 8) + b / 8 (T tiles, padded to a
// multiple of 8): each XCD gets a contiguous run of tiles in row-major
// (m-tile, n-tile) order, i.e. mostly one m-tile, whose A rows then stay in
// that XCD's L2 while its CUs sweep the n-tiles.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "internal.hpp"
#include "lds.hpp"

namespace unillm {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int PBN = 256;         // output columns per workgroup
constexpr int PBK = 64;          // k per step (two blocks)
constexpr int kWaves = 8;        // waves per workgroup (two per SIMD)

__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
    uint32_t r;  // round to nearest even, lo in the low half
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}

// f16 pair (v - bias) * sc, v holding two f16 1024 + code: exact but the last step
__device__ __forceinline__ uint32_t scale2(uint32_t v, f16x2 bias, f16x2 sc) {
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, v) - bias) * sc);
}

// f16 pair (v - bias) * sc - off (Q4_K's and Q5_K's block minimum)
__device__ __forceinline__ uint32_t scale2o(uint32_t v, f16x2 bias, f16x2 sc, f16x2 off) {
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, v) - bias) * sc - off);
}

// One lane's B fragment of one 32-block: its 8 codes (one per byte of `raw`: a
// nibble of each for Q4_0 / Q4_K, selected by `mask`) -> 8 f16 in the order
// 0 2 1 3 4 6 5 7 (x is stored in that order).  (code | 0x6400) is the f16
// 1024 + code exactly; minus `bias` it is the signed code exactly, and times sc =
// d 2^-E it rounds once, as (q - 8) d 2^-E computed in f32 and rounded to f16
// would (E: the weight's exponent offset).
//   Q4_0: a low nibble lands as 1024 + q (bias 1032, sc = d 2^-E), a high nibble
//         in place as 1024 + 16 q (bias 1152, sc = d 2^-E / 16);
//   Q4_K: the same with bias 1024, sc = d sc_b 2^-E (/ 16), minus off = dmin m_b
//         2^-E (sc and off rounded to f16 once each, the weight once more);
//   Q8_0 / Q6_K: a byte (int8 code, flipped to q + 128) as 1024 + q + 128, bias
//         1152 (Q6_K: the code is q - 32, sc = d sc_half 2^-E);
//   Q5_K: a byte (the code q - 16) as 1024 + q - 16 + 128, bias 1136, sc and off as
//         Q4_K's.
// About 1.75 VALU per weight (Q4_K 2.25), against ~3.25 for an fp32 dequant
// rounded to bf16 (this kernel's earlier form).
template <int QT>
__device__ __forceinline__ f16x8 dequant8_f16(u32x2 raw, uint32_t mask, f16x2 bias, f16x2 sc,
                                              f16x2 off) {
    constexpr bool kNib = QT == UNILLM_QTYPE_Q4_0 || QT == UNILLM_QTYPE_Q4_K;
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t p0, p1;
        if constexpr (kNib) {
            // signed nibbles flipped to q under the f16 exponent 0x6400:
            // ((w ^ 0x88888888) & mask) | 0x64006400 as one v_bitop3 each
            const uint32_t kx = (0x88888888u & mask) | 0x64006400u;
            p0 = (raw[h] & mask) ^ kx;           // bytes 0, 2
            p1 = ((raw[h] >> 8) & mask) ^ kx;    // bytes 1, 3
        } else {
            const uint32_t w = raw[h] ^ 0x80808080u;  // int8 -> q + 128
            p0 = __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u);
            p1 = __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u);
        }
        if constexpr (QT == UNILLM_QTYPE_Q4_K || QT == UNILLM_QTYPE_Q5_K) {
            o[2 * h] = scale2o(p0, bias, sc, off);
            o[2 * h + 1] = scale2o(p1, bias, sc, off);
        } else {
            o[2 * h] = scale2(p0, bias, sc);
            o[2 * h + 1] = scale2(p1, bias, sc);
        }
    }
    return __builtin_bit_cast(f16x8, o);
}

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- LDS ring ------------------------------------------------------------------------------
// S stages, each one k step (64 k) of both operands, filled by direct
// global -> LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// lane * 16 of the instruction's 1 KiB destination; no VGPRs involved):
//   A  [BM rows][128 B]  f16 x, swizzled: the 16-byte chunk c of row r sits in
//                        slot c ^ (r % 8), so the 16 rows an MFMA fragment read
//                        touches spread over the banks;
//   Bp [256 cols][32 B]  the step's two payloads of each weight row;
//   Bs [256 cols][4 B]   their two f16 scales (x2: each wave loads 32 columns'
//                        scales with all 64 lanes, the upper half a duplicate).
// The compiler is kept out of the LDS reads (inline asm) so it never inserts
// its conservative "wait for every direct load" before them; the kernel waits
// for exactly the stage it reads (vmcnt counts a wave's loads in issue order)
// and then meets the other waves at a bare s_barrier (no fence: a fence would
// also drain the stages still in flight).

template <int QT, int BM>
struct Ring {
    static constexpr int QB =
        QT == UNILLM_QTYPE_Q8_0 || QT == UNILLM_QTYPE_Q5_K || QT == UNILLM_QTYPE_Q6_K
            ? 32
            : 16;  // payload bytes per block
    static constexpr bool K4 = QT == UNILLM_QTYPE_Q4_K, K6 = QT == UNILLM_QTYPE_Q6_K;
    // K-quants with Q4_K's scale words and minimum: Q4_K, Q5_K
    static constexpr bool KM = K4 || QT == UNILLM_QTYPE_Q5_K;
    static constexpr bool KQ = KM || K6;
    static constexpr int A = BM * 128;
    static constexpr int BP = PBN * 2 * QB;
    static constexpr int BS = 2 * PBN * 4;
    static constexpr int BH = KQ ? 2 * PBN * 4 : 0;  // K-quants: the step's group header per column
    static constexpr int STAGE = A + BP + BS + BH;
    // stages: 4 for 128-row tiles (four fit in LDS; ~10 % over three measured),
    // 3 for 256-row tiles
    static constexpr int STAGES = BM == 128 ? 4 : 3;
    // + the tile's row scales of x (f16 operands): BM floats after the ring
    static constexpr int BYTES = STAGES * STAGE + BM * 4;
    static constexpr int RS = STAGES * STAGE;
    static constexpr int CPB = 2 * QB / 16;            // 16-byte payload chunks per column
    static constexpr int AQ = BM / 8 / 8;              // A loads (8 rows each) per wave
    static constexpr int DMA = AQ + CPB / 2 + 1 + (KQ ? 1 : 0);  // direct loads per wave per stage
};

template <int QT, int BM, int NW>
__global__ __launch_bounds__(NW * 64, 1) void prefill_kernel(const uint8_t* __restrict__ base,
                                                              int64_t rb,
                                                              const uint16_t* __restrict__ xb,
                                                              float* __restrict__ y, int M, int N,
                                                              int KB, int tiles_n, int tiles,
                                                              int units_pad, int S, int add,
                                                              float wscale, float oscale,
                                                              const float* __restrict__ rs,
                                                              float* __restrict__ part) {
    static_assert(NW == 8, "the ring's load split assumes 8 waves");
    constexpr int QB = Ring<QT, BM>::QB;  // payload bytes per block
    // waves: RW row groups x CW column groups; wave (rw, cw) owns rows BM / RW * rw ..
    // and columns PBN / CW * cw .. of the tile; its columns' weights are dequantized
    // by the RW waves of the group.  RW = 1: each weight once, all of A per wave.
    constexpr int RW = 1, CW = NW / RW;
    constexpr int WR = BM / RW;                            // rows per wave
    constexpr int WC = PBN / CW;                           // output columns per wave (32)
    constexpr int TI = WR / 16;                            // MFMA tiles along m per wave
    constexpr int TJ = WC / 16;                            // MFMA tiles along n per wave (2)
    using R = Ring<QT, BM>;
    // f16 operands: x rows in the order 0 2 1 3 4 6 5 7, each scaled by a power of
    // two undone by rs[row]; weights scaled by wscale = 2^-E, undone by oscale = 2^E
    using VT = f16x8;
    constexpr int kStages = R::STAGES;
    constexpr int AQ = R::AQ;
    constexpr int CPB = R::CPB;
    extern __shared__ __attribute__((aligned(16))) uint8_t ring[];

    // ---- work unit (XCD-aware): unit u = (k slice sp, tile t), in (sp, m-tile,
    // n-tile) order ----
    const int per_xcd = units_pad / 8;
    const int u = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (u >= tiles * S) return;  // padding workgroups (uniform: the whole workgroup leaves)
    const int sp = u / tiles, t = u % tiles;
    const int mt = t / tiles_n, nt = t % tiles_n;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = mt * BM, n0 = nt * PBN;
    const uint32_t K = (uint32_t)KB * QK;
    const int ksteps = (KB + 1) / 2;
    // this unit's k steps [ks0, ks0 + nks)
    const int ks0 = (int)((int64_t)sp * ksteps / S);
    const int nks = (int)((int64_t)(sp + 1) * ksteps / S) - ks0;

    // ---- this lane's direct-load sources (k-independent parts) ----
    // A: load q covers tile rows 8 q .. 8 q + 7; lane -> row 8 q + lane / 8, slot lane % 8,
    // global chunk (lane % 8) ^ (row % 8).  Rows past m read row m - 1 (never stored).
    uint32_t arow_off[AQ], achunk[AQ];
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
        const int r = 8 * (wv * AQ + q) + lane / 8;
        achunk[q] = (uint32_t)(((lane % 8) ^ (r % 8)) * 8);
        arow_off[q] = (uint32_t)min(m0 + r, M - 1) * K;
    }
    // B payload: wave wv covers tile columns 32 wv .. +31, CPB chunks each; load u: lane ->
    // column 32 wv + u (64 / CPB) + lane / CPB, chunk c = lane % CPB (block c / (QB / 16),
    // 16-byte half c % (QB / 16)).  Scales: lane -> column 32 wv + lane % 32 (upper half of
    // the wave writes a duplicate).
    uint32_t pcol_off[CPB / 2];
#pragma unroll
    for (int u = 0; u < CPB / 2; ++u)
        pcol_off[u] = (uint32_t)min(n0 + 32 * wv + u * (64 / CPB) + lane / CPB, N - 1) * (uint32_t)rb;
    const int pblk = (lane % CPB) / (QB / 16);
    const uint32_t phalf = (uint32_t)((lane % CPB) % (QB / 16)) * 16;
    const uint32_t ssrc = (uint32_t)min(n0 + 32 * wv + lane % 32, N - 1) * (uint32_t)rb +
                          (uint32_t)KB * QB;

    // direct load q (0 .. R::DMA - 1, in this order) of this wave's loads of step ks
    auto issue_one = [&](int ks, int q) {
        uint8_t* st = ring + (ks % kStages) * R::STAGE;
        if (q < AQ) {
            // k chunks past the end (an odd KB's last step) re-read the row's last
            // chunk: x is finite and those k have zero weights
            dma16(xb + arow_off[q] + min((uint32_t)ks * PBK + achunk[q], K - 8),
                  st + (wv * AQ + q) * 1024);
        } else if (q < AQ + CPB / 2) {
            const int u = q - AQ;
            const uint32_t kb = (uint32_t)min(2 * ks + pblk, KB - 1);
            dma16(base + pcol_off[u] + kb * QB + phalf, st + R::A + wv * (CPB / 2) * 1024 + u * 1024);
        } else if (q == AQ + CPB / 2) {
            // the step's two scales (2 ks is even: one aligned dword; an odd KB's last
            // step reads two bytes past the scales, inside the row padding or the
            // weight's tail slot)
            dma4(base + ssrc + 4u * ks, st + R::A + R::BP + wv * 256);
        } else if constexpr (R::KQ) {
            // K-quants: the 256-weight group header of the step (blocks 2 ks, 2 ks + 1)
            dma4(base + ssrc + 2u * (uint32_t)KB + 4u * (uint32_t)(ks >> 2),
                 st + R::A + R::BP + R::BS + wv * 256);
        }
    };
    auto issue = [&](int ks) {  // all of this wave's R::DMA direct loads of step ks
#pragma unroll
        for (int q = 0; q < R::DMA; ++q) issue_one(ks, q);
    };

    // ---- B fragment geometry: lane -> column 16 j + l % 16 of the wave's 32, elements
    // 8 g .. +7 of a block (g = l / 16): Q4_0 payload bytes 8 (g & 1) .. +7, low nibbles
    // for g < 2, high for g >= 2; Q8_0 bytes 8 g .. +7
    const int g = lane / 16, fr = lane % 16;
    constexpr bool kNib = QB == 16;
    const uint32_t boff = kNib ? 8 * (g & 1) : 8 * g;
    const int rw = wv / CW, cw = wv % CW;
    bool bval[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) bval[j] = n0 + WC * cw + 16 * j + fr < N;
    // f16 dequant constants of this lane (high nibbles: 1024 + 16 q, scale / 16)
    const bool hnib = kNib && g >= 2;
    const uint32_t nmask = hnib ? 0x00F000F0u : 0x000F000Fu;
    const _Float16 bias1 = (_Float16)(QT == UNILLM_QTYPE_Q4_K                 ? 1024.0f
                                      : QT == UNILLM_QTYPE_Q5_K               ? 1136.0f
                                      : QT == UNILLM_QTYPE_Q4_0 && !hnib ? 1032.0f
                                                                         : 1152.0f);
    const float lsc = hnib ? 0.0625f : 1.0f;
    const f16x2 fbias = {bias1, bias1};
    float wl[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) wl[j] = bval[j] ? (hnib ? wscale * 0.0625f : wscale) : 0.0f;
    // LDS byte offsets (within a stage) of this lane's reads; the row tile i and the
    // column tile j enter as immediate offsets.  A: row WR rw + 16 i + fr, chunk
    // 4 kk + g in slot (4 kk + g) ^ (row % 8), and row % 8 == fr % 8.
    uint32_t aoff[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
        aoff[kk] = (uint32_t)((WR * rw + fr) * 128 + (((4 * kk + g) ^ (fr % 8)) * 16));
    // B payload of column WC cw + 16 j + fr: block b at b * QB + boff; its scales
    // (column c at (c / 32) * 256 + (c % 32) * 4)
    const int bc0 = WC * cw + fr;
    const uint32_t boff0 = (uint32_t)(R::A + bc0 * (2 * QB) + boff);
    const uint32_t soff0 = (uint32_t)(R::A + R::BP + (bc0 / 32) * 256 + (bc0 % 32) * 4);
    const uint32_t ring0 = (uint32_t)(uintptr_t)ring;

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // prologue: the tile's row scales (f16 operands; wave 0, ahead of its ring loads, so
    // the ring's waits cover them), then stages 0 .. kStages - 2 in flight
    if (wv == 0) {
#pragma unroll
        for (int q = 0; q < BM / 64; ++q)
            dma4(rs + min(m0 + 64 * q + lane, M - 1), ring + R::RS + q * 256);
    }
#pragma unroll
    for (int d = 0; d < kStages - 1; ++d)
        if (d < nks) issue(ks0 + d);

    for (int j = 0; j < nks; ++j) {
        const int ks = ks0 + j;
        // wait for this wave's loads of step ks: the loads of later steps already
        // issued (at most kStages - 2 of them) may stay in flight
        // (min(kStages - 2, nks - 1 - j) younger steps in flight: the full count, one
        // or none at the end)
        if (j + kStages - 2 < nks) wait_vmcnt<(kStages - 2) * R::DMA>();
        else if (j + 1 < nks) wait_vmcnt<R::DMA>();
        else wait_vmcnt<0>();
        const uint32_t st = ring0 + (uint32_t)((ks % kStages) * R::STAGE);
        // B: raw bytes and scales (K-quants: and group headers) of this wave's columns.
        // They are this wave's own loads, complete after the wait above, so they are
        // read before the barrier: the reads' latency passes while the waves meet.
        // Raw payload of column tile j at j * 16 * 2 QB (block 1 at + QB); scales of
        // tile j at (16 j / 32) * 256 + (16 j % 32) * 4 relative to tile 0's
        static_assert(TJ == 2, "two column tiles");
        constexpr int T = 16 * 2 * QB;
        u32x2 raw[TJ][2];
        uint32_t sc[TJ], hd[TJ];
        asm volatile(
            "ds_read_b64 %0, %6 offset:%c8\n ds_read_b64 %1, %6 offset:%c9\n"
            "ds_read_b64 %2, %6 offset:%c10\n ds_read_b64 %3, %6 offset:%c11\n"
            "ds_read_b32 %4, %7\n ds_read_b32 %5, %7 offset:64"
            : "=&v"(raw[0][0]), "=&v"(raw[0][1]), "=&v"(raw[1][0]), "=&v"(raw[1][1]), "=&v"(sc[0]),
              "=&v"(sc[1])
            : "v"(st + boff0), "v"(st + soff0), "i"(0), "i"(QB), "i"(T), "i"(T + QB));
        if constexpr (R::KQ)
            asm volatile("ds_read_b32 %0, %2\n ds_read_b32 %1, %2 offset:64"
                         : "=&v"(hd[0]), "=&v"(hd[1])
                         : "v"(st + soff0 + R::BS));
        __builtin_amdgcn_s_barrier();
        if constexpr (R::KQ)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(raw[0][0]), "+v"(raw[0][1]), "+v"(raw[1][0]), "+v"(raw[1][1]),
                           "+v"(sc[0]), "+v"(sc[1]), "+v"(hd[0]), "+v"(hd[1]));
        else
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(raw[0][0]), "+v"(raw[0][1]), "+v"(raw[1][0]), "+v"(raw[1][1]),
                           "+v"(sc[0]), "+v"(sc[1]));
        // the loads of step ks + kStages - 1 are issued spread over this step's MFMAs
        // (after fragments 0, SPC, 2 SPC, ..), not all at once: their data then reaches
        // LDS spread over the step rather than in one burst among the fragment reads
        const bool issue_next = j + kStages - 1 < nks;

        const bool b1ok = 2 * ks + 1 < KB;
        // the f16 scales of blocks 0 (low half) and 1 (high half) of each column tile,
        // and Q4_K's offsets
        uint32_t sp[TJ], op[TJ];
        if constexpr (!R::KQ) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                sp[j] = pack_f16(__half2float(__ushort_as_half((uint16_t)sc[j])) * wl[j],
                                 b1ok ? __half2float(__ushort_as_half((uint16_t)(sc[j] >> 16))) * wl[j]
                                      : 0.0f);
                op[j] = 0;
            }
        } else {
            // the group header (Q4_K, Q5_K d | dmin << 16, Q6_K d) of each column tile, laid out
            // as the scales; sc[j] holds block 0's u16 in its low half, block 1's in its
            // high: Q4_K, Q5_K sc | m << 8, Q6_K the int8 scales of the two 16-weight halves
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const float dd =
                    bval[j] ? __half2float(__ushort_as_half((uint16_t)hd[j])) * wscale : 0.0f;
                if constexpr (R::KM) {
                    const float dm =
                        bval[j] ? __half2float(__ushort_as_half((uint16_t)(hd[j] >> 16))) * wscale
                                : 0.0f;
                    sp[j] = pack_f16(dd * (float)(sc[j] & 0xFFu) * lsc,
                                     b1ok ? dd * (float)((sc[j] >> 16) & 0xFFu) * lsc : 0.0f);
                    op[j] = pack_f16(dm * (float)((sc[j] >> 8) & 0xFFu),
                                     b1ok ? dm * (float)(sc[j] >> 24) : 0.0f);
                } else {
                    // this lane's elements 8 g .. 8 g + 7 lie in half g / 2 of each block
                    const int hs = 8 * (g >> 1);
                    sp[j] = pack_f16(dd * (float)(int8_t)(sc[j] >> hs),
                                     b1ok ? dd * (float)(int8_t)(sc[j] >> (16 + hs)) : 0.0f);
                    op[j] = 0;
                }
            }
        }
        auto deq = [&](int j, int b) -> VT {
            const f16x2 s2 = __builtin_bit_cast(f16x2, sp[j]), o2 = __builtin_bit_cast(f16x2, op[j]);
            const f16x2 sb = b == 0 ? f16x2{s2[0], s2[0]} : f16x2{s2[1], s2[1]};
            const f16x2 ob = b == 0 ? f16x2{o2[0], o2[0]} : f16x2{o2[1], o2[1]};
            return dequant8_f16<QT>(raw[j][b], nmask, fbias, sb, ob);
        };
        // block 0's fragments first; block 1's are dequantized between the MFMAs of
        // the first 32 k (one column tile after every TI / TJ row tiles), so the
        // VALU work overlaps the matrix cores instead of following them
        VT bfrag[TJ][2];
#pragma unroll
        for (int j = 0; j < TJ; ++j) bfrag[j][0] = deq(j, 0);
        // A fragments, two ahead (one ahead leaves ~2 MFMAs to cover an LDS read;
        // deeper measured no better): fragment f = kk * TI + i at aoff[kk] + 2048 i
        constexpr int PF = 2;
        VT afr[2 * TI];
        constexpr_for<PF>([&](auto F) {
            afr[F.value] = __builtin_bit_cast(
                VT, lds_read128<(F.value % TI) * 2048>(st + aoff[F.value / TI]));
        });
#pragma unroll
        for (int f = 0; f < 2 * TI; ++f) {
            if (f + PF < 2 * TI) {
                constexpr_for<2 * TI>([&](auto F) {
                    if (F.value == f + PF)
                        afr[F.value] = __builtin_bit_cast(
                            VT, lds_read128<(F.value % TI) * 2048>(st + aoff[F.value / TI]));
                });
                asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(afr[f]));
            } else if (f + 1 < 2 * TI) {
                asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(afr[f]));
            } else {
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(afr[f]));
            }
            const int kk = f / TI, i = f % TI;
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = mfma16(afr[f], bfrag[j][kk], acc[i][j]);
            if (kk == 0 && (i + 1) % (TI / TJ) == 0) {
                const int j = (i + 1) / (TI / TJ) - 1;
                bfrag[j][1] = deq(j, 1);
            }
            constexpr int SPC = 2 * TI / R::DMA;  // fragments between two loads
            static_assert(SPC >= 1, "a load slot for every direct load");
            if (issue_next && f % SPC == 0 && f / SPC < R::DMA) issue_one(ks + kStages - 1, f / SPC);
        }
    }

    // ---- epilogue: lane holds C[4 (l / 16) + e][l % 16] of each 16 x 16 tile.  One
    // k slice (S = 1): f16 operands, so the output factor of row 16 i + 4 g + e is
    // oscale times its row scale (from LDS: global loads here would wait for the
    // stores before them).  S slices: each stores its raw sums to its slab of `part`
    // ([S][M][N]); split_sum_kernel adds the slabs in slice order and scales them ----
    if (S > 1) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + WC * cw + 16 * j + fr;
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = m0 + WR * rw + 16 * i + 4 * g + e;
                    if (row < M) part[((int64_t)sp * M + row) * N + col] = acc[i][j][e];
                }
        }
        return;
    }
    float4 rsc[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const float4 r4 =
            *reinterpret_cast<const float4*>(ring + R::RS + (WR * rw + 16 * i + 4 * g) * 4);
        rsc[i] = make_float4(r4.x * oscale, r4.y * oscale, r4.z * oscale, r4.w * oscale);
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = n0 + WC * cw + 16 * j + fr;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + WR * rw + 16 * i + 4 * g + e;
                if (row >= M) continue;
                float* dst = y + (int64_t)row * N + col;
                const float v =
                    acc[i][j][e] * (e == 0 ? rsc[i].x : e == 1 ? rsc[i].y : e == 2 ? rsc[i].z : rsc[i].w);
                *dst = add ? *dst + v : v;
            }
    }
}

// y[r, c] (+)= (sum over the S slabs of part[s][r][c], in slice order) * rs[r] * oscale:
// the k slices of a split prefill, in a fixed order (the result does not depend on
// which slice finished first).  Four columns a thread when vec (n % 4 == 0 and y on
// a 16-byte boundary).
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ part, int S,
                                                        int64_t M, int64_t N,
                                                        const float* __restrict__ rs,
                                                        float oscale, int add, int vec,
                                                        float* __restrict__ y) {
    const int64_t MN = M * N;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (vec) {
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < MN / 4; q += stride) {
            f32x4 v = *reinterpret_cast<const f32x4*>(part + 4 * q);
            for (int sl = 1; sl < S; ++sl)
                v += *reinterpret_cast<const f32x4*>(part + sl * MN + 4 * q);
            v *= rs[4 * q / N] * oscale;
            f32x4* dst = reinterpret_cast<f32x4*>(y + 4 * q);
            *dst = add ? *dst + v : v;
        }
        return;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += stride) {
        float v = part[i];
        for (int sl = 1; sl < S; ++sl) v += part[sl * MN + i];
        v *= rs[i / N] * oscale;
        y[i] = add ? y[i] + v : v;
    }
}

// x is addressed with 32-bit element offsets: a launch takes at most this many rows
int64_t prefill_chunk_rows(int64_t k, int bm) {
    return std::max<int64_t>(bm, ((int64_t)1 << 30) / k / bm * bm);
}

template <int QT, int BM>
hipError_t launch_bm(const QWeight& w, const uint16_t* xb, const float* rs, int64_t m, float* y,
                     int S, float* part, hipStream_t s, int add) {
    const int64_t chunk = prefill_chunk_rows(w.k, BM);
    if (m > chunk) {  // row chunks below 2^30 elements (the plan never splits k here)
        if (S != 1) return hipErrorInvalidValue;
        for (int64_t r = 0; r < m; r += chunk) {
            hipError_t e =
                launch_bm<QT, BM>(w, xb + r * w.k, rs ? rs + r : nullptr, std::min(chunk, m - r),
                                  y + r * w.n, 1, nullptr, s, add);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    static bool attr = [] {
        return hipFuncSetAttribute((const void*)prefill_kernel<QT, BM, kWaves>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   Ring<QT, BM>::BYTES) == hipSuccess;
    }();
    if (!attr) return hipErrorInvalidValue;
    const int tiles_m = (int)((m + BM - 1) / BM);
    const int tiles_n = (int)((w.n + PBN - 1) / PBN);
    const int tiles = tiles_m * tiles_n;
    const int units_pad = (tiles * S + 7) / 8 * 8;
    const float wscale = ldexpf(1.0f, -w.f16_exp), oscale = ldexpf(1.0f, w.f16_exp);
    prefill_kernel<QT, BM, kWaves><<<units_pad, kWaves * 64, Ring<QT, BM>::BYTES, s>>>(
        w.base, w.row_bytes, xb, y, (int)m, (int)w.n, (int)w.kb, tiles_n, tiles, units_pad, S,
        add, wscale, oscale, rs, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int vec = w.n % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    const int64_t q = m * w.n / (vec ? 4 : 1);
    const int blocks = (int)std::min<int64_t>((q + 255) / 256, 8 * device_info().cu_count);
    split_sum_kernel<<<blocks, 256, 0, s>>>(part, S, m, w.n, rs, oscale, add, vec, y);
    return hipGetLastError();
}

// Tile rows and k split.  256-row tiles when they give at least one tile per CU,
// unless 128-row tiles take no more rounds.
// A deep product (128 k steps or more) whose 256-row tiles fill at most half the
// CUs takes those tiles with the k steps split over up to CUs / tiles workgroups, at
// least 16 steps each: where the tiles fill 3/8 to 1/2 of the CUs (a split in two:
// m2048 k14336 n4096, 128 tiles, 256 workgroups; Q4_0 776-796 -> 866 TFLOP/s a call,
// Q8_0 759-774 -> 897-902 against one 128-row tile a CU), and for m > 256 where
// plan_cost rates them no dearer than the 128-row plan (m1024 k14336 n4096, 64 tiles in
// 4 slices: Q4_0 163-169 -> 154-156 us a call against 128 tiles of 128 rows in 2;
// m768, 48 tiles in 5: 159-161 -> 126-127).  Else 128-row tiles; when those fill at
// most half the CUs (a short, deep product), the k steps are split over up to 16
// workgroups per tile, at least 8 steps each; unless (m > 256) plan_cost rates the
// 256-row tiles unsplit cheaper.  Split slices' raw sums meet in
// split_sum_kernel (slabs of the stream's workspace).  Calls beyond the 32-bit x
// offsets (chunked) never split.
struct PrefillPlan {
    int bm, S;
};
// the most 128-row tiles that split their k steps: half the CUs or fewer
int64_t split_tiles_max() { return device_info().cu_count / 2; }
// the most slices a k range splits into
constexpr int64_t kMaxSlices = 16;
size_t up256(size_t b) { return (b + 255) / 256 * 256; }

// The workspace a plan takes: x as f16 rows | their scales | the split slabs
// ([S][m][n] f32)
size_t plan_bytes(const QWeight& w, int64_t m, int S) {
    const size_t slabs = S > 1 ? (size_t)S * m * w.n * sizeof(float) : 0;
    return up256((size_t)m * (size_t)w.k * 2) + up256((size_t)m * sizeof(float)) + slabs;
}

// The busiest CU's share of a plan: rounds x rows x k steps a workgroup, a 128-row
// tile's rows counted at 8/7 of a 256-row tile's (770 against 889 TFLOP/s a kernel,
// Q4_0 m512 and m2048 at k4096 n14336, unsplit)
int64_t plan_cost(int64_t tiles, int64_t S, int bm, int64_t ksteps, int64_t cus) {
    const int64_t rounds = (tiles * S + cus - 1) / cus;
    return rounds * bm * ((ksteps + S - 1) / S) * (bm == 128 ? 8 : 7);
}

// cap > 0: a caller's fixed workspace of cap bytes; a split plan that does not fit
// falls back to a plan that does (at worst the 128-row tiles unsplit)
PrefillPlan prefill_plan(const QWeight& w, int64_t m, size_t cap = 0) {
    const int64_t cus = device_info().cu_count;
    const int64_t tiles_n = (w.n + PBN - 1) / PBN;
    const int64_t t256 = (m + 255) / 256 * tiles_n;
    const int64_t ksteps = (w.kb + 1) / 2;
    const int64_t tiles = (m + 127) / 128 * tiles_n;
    // a tile a CU or more: 128-row tiles where they take no more rounds, each half
    // as long (k4096 n14336 m1100: 504 tiles against 280, two rounds each; Q4_0
    // 233 -> 187-189 us a call, Q8_0 231-233 -> 205-207; a third round loses)
    if (t256 >= cus)
        return (tiles + cus - 1) / cus <= (t256 + cus - 1) / cus ? PrefillPlan{128, 1}
                                                                 : PrefillPlan{256, 1};
    int64_t S = 1;
    if (tiles <= split_tiles_max() && m <= prefill_chunk_rows(w.k, 128))
        S = std::max<int64_t>(1, std::min<int64_t>({kMaxSlices, cus / tiles, ksteps / 8}));
    if (S > 1 && cap > 0 && plan_bytes(w, m, (int)S) > cap) S = 1;
    if (ksteps >= 128 && 2 * t256 <= cus && m <= prefill_chunk_rows(w.k, 256)) {
        const int64_t S2 = std::min<int64_t>({kMaxSlices, cus / t256, ksteps / 16});
        const bool cheaper =
            m > 256 && plan_cost(t256, S2, 256, ksteps, cus) <= plan_cost(tiles, S, 128, ksteps, cus);
        if ((8 * t256 >= 3 * cus || cheaper) && (cap == 0 || plan_bytes(w, m, (int)S2) <= cap))
            return {256, (int)S2};
    }
    // fewer 256-row tiles than CUs, but one round of them against two of 128-row
    // tiles (k4096 n14336 m1024: 224 tiles against 448; Q4_0 166-171 -> 134 us a
    // call, 20-25 % on every shape it picks)
    if (m > 256 && plan_cost(t256, 1, 256, ksteps, cus) < plan_cost(tiles, S, 128, ksteps, cus))
        return {256, 1};
    return {128, (int)S};
}

}  // namespace

// The call's own need (for a caller's fixed workspace of cap bytes, cap > 0, the
// plan that fits it where one does), and a bound for every m' <= m (the slabs of 4
// slices of the largest m' that can split), so that a reserve for m covers every
// shorter call.
size_t prefill_call_bytes(const QWeight& w, int64_t m, size_t cap) {
    return plan_bytes(w, m, prefill_plan(w, m, cap).S);
}

size_t prefill_workspace_bytes(const QWeight& w, int64_t m) {
    // slices x rows of any split: at most kMaxSlices m, and at most 128 CUs / (column
    // tiles) with 128-row tiles (S <= CUs / tiles) or 256 CUs / (column tiles) with
    // 256-row tiles (S <= CUs / tiles)
    const int64_t tiles_n = (w.n + PBN - 1) / PBN;
    const int64_t sm = (w.kb + 1) / 2 < 16
                           ? 0  // fewer than 2 x 8 k steps: never split
                           : std::min<int64_t>(kMaxSlices * m,
                                               256 * device_info().cu_count / tiles_n);
    const size_t slabs = (size_t)sm * w.n * sizeof(float);
    return up256((size_t)m * (size_t)w.k * 2) + up256((size_t)m * sizeof(float)) + slabs;
}

hipError_t launch_prefill_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                               hipStream_t s, int epi, const NormArgs& norm, void* ws,
                               size_t ws_bytes) {
    // weight bytes are addressed with 32-bit offsets (pcol_off, ssrc)
    if (!mfma_supports(w)) return hipErrorInvalidValue;
    // x as f16 rows with their power-of-two scales in the workspace: the GEMM
    // re-reads x once per 256-column tile, so it reads half the bytes, and no
    // conversion sits in its inner loop.  A split k's slabs follow.
    const PrefillPlan plan = prefill_plan(w, m, ws ? ws_bytes : 0);
    const size_t xbytes = up256((size_t)m * (size_t)w.k * 2);
    hipError_t e = hipSuccess;
    if (ws && plan_bytes(w, m, plan.S) > ws_bytes) return hipErrorInvalidValue;
    if (!ws && (e = stream_workspace(s, plan_bytes(w, m, plan.S), &ws)) != hipSuccess) return e;
    float* rs = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + xbytes);
    float* part =
        plan.S > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + xbytes +
                                              up256((size_t)m * sizeof(float)))
                   : nullptr;
    const int add = epi == kEpiAdd;
    e = norm.gamma ? launch_norm_convert(x, m, w.k, norm, ws, y, 0, s, rs)
                   : launch_x_to_f16_rows(x, m, w.k, ws, rs, s);
    if (e != hipSuccess) return e;
    const uint16_t* xb = static_cast<const uint16_t*>(ws);
#define UNILLM_PREFILL_LAUNCH(QTYPE)                                                          \
    return plan.bm == 256 ? launch_bm<QTYPE, 256>(w, xb, rs, m, y, plan.S, part, s, add)     \
                          : launch_bm<QTYPE, 128>(w, xb, rs, m, y, plan.S, part, s, add)
    switch (w.qtype) {
        case UNILLM_QTYPE_Q4_0: UNILLM_PREFILL_LAUNCH(UNILLM_QTYPE_Q4_0);
        case UNILLM_QTYPE_Q8_0: UNILLM_PREFILL_LAUNCH(UNILLM_QTYPE_Q8_0);
        case UNILLM_QTYPE_Q4_K: UNILLM_PREFILL_LAUNCH(UNILLM_QTYPE_Q4_K);
        case UNILLM_QTYPE_Q5_K: UNILLM_PREFILL_LAUNCH(UNILLM_QTYPE_Q5_K);
        case UNILLM_QTYPE_Q6_K: UNILLM_PREFILL_LAUNCH(UNILLM_QTYPE_Q6_K);
        default: return hipErrorInvalidValue;
    }
#undef UNILLM_PREFILL_LAUNCH
}

}  // namespace unillm
