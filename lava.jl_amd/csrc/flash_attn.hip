// flash_attn.hip -- causal flash-attention forward, fp16 in/out, fp32 softmax state.
//
// The reference is the coopmat2 flash kernel Lava's vocabulary was shaped for
// (`attn_flash_rows!` / flash_attn_cm2, src/vocabulary/coopmat.jl:158;
// src/device/coopmat_intrinsics.jl:535-755): per query block, per key block,
//   S = Q K^T; rowmax = reduce(max, S, Row); M = max(rowmax, Mold);
//   P = exp(S - M); O = O * exp(Mold - M) + P V; L = L * exp(Mold - M) + rowsum(P)
// and finally O / L, converted to fp16 (RNE).
//
// Kernels (the dispatcher at the end of the file picks one):
//  * flash_fwd5_kernel -- D <= 128 (the headline shape D = 128), any softmax scale: on each SIMD
//    a score wavefront and an output wavefront share 64 queries (described at the kernel);
//  * flash_fwd3_kernel -- D = 256 with a positive scale (and D = 64 or 128 on request):
//    ping-pong pairs of 32-query wavefronts;
//  * flash_generic_kernel -- any D <= 256, one thread per query (every other case).
//
// The common CDNA4 formulation:
//  * everything is computed transposed, S^T = K Q^T and O^T = V^T P^T, on the 32x32x16
//    fp16 MFMA.  In that form the accumulator lane owns ONE query (lane % 32; lanes l and
//    l ^ 32 share it) and holds that query's scores for 16 keys per 32-key tile, so the row
//    max and row sum are in-lane reductions plus one exchange with lane ^ 32, the rescale of
//    O is one multiplier per lane, and the score accumulator converts in place to the B
//    operand P^T of the second product (keys in-lane), with no relayout;
//  * Q^T stays in registers for the whole key loop;
//  * K and V blocks of 64 keys are staged in LDS by LDS-DMA, 16-byte chunks XOR-swizzled so
//    that the K fragment reads and the transposing V reads are bank-conflict-free;
//  * softmax in base 2 (s * scale * log2 e, v_exp_f32) with lazy rescaling;
//  * causal: key blocks above the diagonal are never loaded, and only the diagonal block is
//    masked per element;
//  * workgroups are ordered XCD by XCD so that all query blocks of one (batch, head) run on
//    one XCD and share its K and V through that XCD's L2; causal: longest query blocks first
//    across groups of the XCD's heads (fa_order).
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "lava_coopmat.hpp"
#include "lava_hip_internal.hpp"
#include "lds_dma.hpp"

namespace lava {

constexpr int FA_D = 128;

struct FaParams {
    const f16* Q;
    const f16* K;
    const f16* V;
    f16* O;
    int64_t sl, sh, sb;      // strides of L, H, B (elements) for Q/K/V
    int64_t osl, osh, osb;   // for O
    int S, H, B;
    float scale_log2;        // softmax scale * log2(e)
    int causal;
    int o16;                 // O and its strides allow 16-byte row stores
    int D;                   // head dimension (the score/output kernel zero-pads it to 128)
    int dv;                  // the ping-pong kernel at DQK = 256: V / O columns of this launch's half
};

// Workgroup -> (batch * head, query block).  Workgroups are dispatched round-robin
// over the 8 XCDs (blockIdx % 8).  Non-causal: every block costs the same, and each
// XCD takes a contiguous range of (head, block) pairs, so one head's K and V stay in
// one XCD's L2.  Causal: query block qb costs qb + 1 key blocks, so each XCD takes
// whole heads (when 8 divides B * H), in groups of 4 heads (when 4 divides the
// XCD's count), and runs a group's heaviest blocks first, then the next lighter
// ones: longest first across the group keeps the dispatch tail short, and one
// group's K and V (8 MiB at D = 128, S = 4096) is what the XCD streams at a time.
// Measured at B = 4, H = 32, S = 4096: groups of 4 heads 934-937 TFLOP/s, of all 16
// of the XCD's heads 886-893, one head at a time 835.  Without the split by XCD,
// heavy first over all heads.
__device__ __forceinline__ void fa_order(int nqb, int nbh, bool causal, int& bh, int& qb) {
    const int bid = blockIdx.x;
    if (causal) {
        if ((nbh & 7) == 0) {
            const int h8 = nbh >> 3, local = bid >> 3;
            const int G = (h8 & 3) == 0 ? 4 : h8;   // heads per group
            const int grp = local / (G * nqb), r = local % (G * nqb);
            qb = nqb - 1 - r / G;
            bh = (bid & 7) * h8 + grp * G + r % G;
        } else {
            qb = nqb - 1 - bid / nbh;
            bh = bid % nbh;
        }
    } else {
        const int total = nqb * nbh;
        const int b2 = (total & 7) == 0 ? (bid & 7) * (total >> 3) + (bid >> 3) : bid;
        bh = b2 / nqb;
        qb = b2 % nqb;
    }
}

// ---------------------------------------------------------------------------
// Version 3 (the fast path): 8 wavefronts x 32 queries = 256 queries per
// workgroup; K and V blocks of 64 keys move global -> LDS by buffer_load ... lds,
// so no VGPRs stage them and each block is loaded once per 256 queries; V^T
// operands come from the row-major V tile through ds_read_b64_tr_b16.
//
// Ping-pong schedule.  Each wavefront alternates an MFMA phase (O += V^T P^T for
// the previous block, then S^T = K Q^T for this one: 32 MFMAs) and a softmax
// phase (VALU only), with a workgroup barrier after every phase.  Wavefronts 4-7
// start one phase late, so each SIMD (holding wavefronts w and w + 4) always has
// one wavefront in its MFMA phase and the other in its softmax phase, and the
// matrix core and the VALU work at the same time instead of taking turns.
//
// K and V have three LDS stages each.  The MFMA phase of iteration kb issues the
// DMA of K block kb + 2 and V block kb + 1 (4 instructions per wavefront at D = 128,
// 6 with 512-byte K rows) and each phase ends with s_waitcnt vmcnt(that count), so a
// wavefront's DMAs have landed by the end of its next MFMA phase; the barrier after
// it publishes them.  The stage a DMA
// overwrites was last read by the late wavefronts one phase before it is issued.
//
// LDS layout: K [64 keys][256 B] and V [64 keys][256 B] per stage, 16-byte chunks
// XOR-swizzled -- K by key % 16 (a fragment read is 32 keys x one chunk), V by
// 4 (key % 4) (a transposing read is 4 keys x 32 bytes per 16-lane group) -- so
// neither read pattern has bank conflicts.
//
// ds_read_b64_tr_b16: in a 16-lane group, output lane i value j is the 16-bit word
// at (address of source lane 4 j + i / 4) + 2 (i % 4).  Source lane 4 jj + q points
// at V[key0 + jj][d0 + 4 q], so output lane i receives V[key0 .. key0 + 3][d0 + i]:
// four keys of one head-dimension column, the k-slots of the V^T operand.
//
// Lazy rescaling: the running maximum moves (and O, L are rescaled) only when a
// block's maximum exceeds it by more than 2^8; P = exp2(s - m) then stays <= 256,
// exact enough in fp16, and O / L is unchanged in exact arithmetic.
constexpr int F3_WAVES = 8;
constexpr int F3_BQ = 32 * F3_WAVES;        // 256 queries per workgroup
constexpr int F3_BK = 64;
constexpr int F3_STAGES = 3;
constexpr float F3_RESCALE = 8.0f;
constexpr int F3_PREFETCH = 4;        // MFMA-phase operations between an LDS read and its use

template <bool B>
struct f3_tag {
    static constexpr bool value = B;
};

typedef short f3_s16x4 __attribute__((ext_vector_type(4)));
typedef short f3_s16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f3_s16x4 f3_read_tr(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) f3_s16x4*)(const __attribute__((address_space(3))) uint8_t*)p);
}

// Asm uses (a comment: the backend drops empty asm) that pin a value's computation before this point: without them the
// compiler sinks the softmax's exp / convert / sum (used only by the next phase's
// MFMAs) across the barrier into the MFMA phase, which undoes the ping-pong.
__device__ __forceinline__ void f3_pin(const f16x8& v) {
    const uint4 u = __builtin_bit_cast(uint4, v);
    asm volatile("; pin" ::"v"(u.x), "v"(u.y), "v"(u.z), "v"(u.w));
}
__device__ __forceinline__ void f3_pin(const f32x16& v) {
#pragma unroll
    for (int i = 0; i < 16; i += 4) asm volatile("; pin" ::"v"(v[i]), "v"(v[i + 1]), "v"(v[i + 2]), "v"(v[i + 3]));
}

// All waits for the DMAs of the phase before last (N = the DMA instructions one
// phase issues), then the workgroup barrier.
template <int N>
__device__ __forceinline__ void f3_phase_end() {
    static_assert(N == 6 || N == 4 || N == 2, "K + V DMA instructions per wavefront and phase");
    if constexpr (N == 6)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else if constexpr (N == 4)
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    __syncthreads();
}

// DQK (the Q / K head dimension: 64, 128 or 256) and DV (the V / O one: 64 or 128; DQK = 256
// runs with DV = 128, once per half of V's columns) set the row sizes (D * 2 bytes = CH chunks
// of 16 bytes), the number of S^T k-steps (DQK / 16) and of O^T row tiles (DV / 32), and the
// swizzles: K chunk ^ (key % 16) for rows of 16 or more chunks, ^ ((key % 8) ^ (key / 8 % 2))
// for 8-chunk rows (a fragment read, 32 keys x one chunk, spread over the banks); V chunk
// ^ 4 (key % 4), resp. ^ 2 (key % 4) (a transposing read, 4 keys x 2 chunks per 16-lane group).
template <bool CAUSAL, int DQK, int DV>
__global__ void __launch_bounds__(64 * F3_WAVES, 1) flash_fwd3_kernel(FaParams p) {
    static_assert((DQK == DV && (DV == 128 || DV == 64)) || (DQK == 256 && DV == 128),
                  "head dimensions 64, 128, or 256 for Q/K with 128 for V/O");
    constexpr int RBK = DQK * 2, RBV = DV * 2;             // bytes per K / V row
    constexpr int CHK = RBK / 16, CHV = RBV / 16;          // 16-byte chunks per row
    constexpr int TILEK = F3_BK * RBK, TILEV = F3_BK * RBV;   // one K / V block
    constexpr int NKS = DQK / 16;                          // S^T MFMAs per key tile
    constexpr int NDT = DV / 32;                           // O^T row tiles
    constexpr int NPV = 4 * NDT;                           // O^T MFMAs per block
    constexpr int NOPS = NPV + 2 * NKS;                    // MFMAs of a full phase
    constexpr int DPTK = TILEK / (1024 * F3_WAVES);        // DMA instructions per wavefront per tile
    constexpr int DPTV = TILEV / (1024 * F3_WAVES);
    constexpr int RPIK = 64 / CHK, RPIV = 64 / CHV;        // rows per DMA instruction
    // LDS operand reads ahead of their MFMA (3 at DQK = 256, where the 16 Q^T fragments fill the
    // registers)
    constexpr int PREF = DQK == 256 ? 3 : F3_PREFETCH;
    __shared__ __attribute__((aligned(1024))) uint8_t kbuf[F3_STAGES][TILEK];   // [stage][key][RBK]
    __shared__ __attribute__((aligned(1024))) uint8_t vbuf[F3_STAGES][TILEV];
    auto kswz = [](int row) { return CHK >= 16 ? (row & 15) : ((row & 7) ^ ((row >> 3) & 1)); };
    auto vswz = [](int row) { return CHV == 16 ? 4 * (row & 3) : 2 * (row & 3); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool late = w >= F3_WAVES / 2;        // one phase behind its SIMD partner w - 4
    const int nqb = (p.S + F3_BQ - 1) / F3_BQ;   // the last query block may be partial
    const int nbh = p.H * p.B;
    int bh, qb;
    fa_order(nqb, nbh, CAUSAL, bh, qb);
    const int hh = bh % p.H, bb = bh / p.H;
    const int64_t head = (int64_t)hh * p.sh + (int64_t)bb * p.sb;
    f16* Ob = p.O + (int64_t)hh * p.osh + (int64_t)bb * p.osb;

    const int q0 = qb * F3_BQ + w * 32;         // this wave's first query
    const int r32 = lane & 31, h = lane >> 5;
    const int my_q = q0 + r32;

    // Q^T as B operand: lane (query my_q, half h) holds d = 16 ks + 8 h + [0, 8);
    // queries past S (a ragged last block) compute on zeros and are not stored
    f16x8 qf[NKS];
    {
        const f16* qrow = p.Q + head + (int64_t)my_q * p.sl + 8 * h;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qf[ks] = f16x8{};
        if (my_q < p.S) {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                if (DQK != 256 || 16 * ks + 8 * h < p.D) qf[ks] = *reinterpret_cast<const f16x8*>(qrow + 16 * ks);
        }
    }

    // ---- LDS-DMA: wave w moves rows [8 w, 8 w + 8) of a K (V) tile in DPTK (DPTV)
    // instructions: instruction i covers rows 8 w + RPI i + lane / CH, physical chunk lane % CH.
    const uint32_t row_bytes = (uint32_t)(p.sl * 2);
    const v4i rk = make_rsrc(p.K + head, (uint32_t)p.S * row_bytes);
    const v4i rv = make_rsrc(p.V + head, (uint32_t)p.S * row_bytes);
    uint32_t voff_k[DPTK], voff_v[DPTV];
    // At DQK = 256 a head dimension D < 256 is zero-padded: a lane whose logical chunk lies at or
    // past D (K) or past this launch's dv columns (V) takes an offset beyond the resource, so the
    // DMA writes zeros (zero K columns add nothing to the scores; zero V columns give O columns
    // that are not stored).
#pragma unroll
    for (int i = 0; i < DPTK; ++i) {
        const int row = 8 * w + RPIK * i + lane / CHK;
        const int c = (lane % CHK) ^ kswz(row);
        voff_k[i] = (DQK != 256 || 8 * c < p.D) ? (uint32_t)row * row_bytes + 16u * (uint32_t)c : 0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < DPTV; ++i) {
        const int row = 8 * w + RPIV * i + lane / CHV;
        const int c = (lane % CHV) ^ vswz(row);
        voff_v[i] = (DQK != 256 || 8 * c < p.dv) ? (uint32_t)row * row_bytes + 16u * (uint32_t)c : 0x80000000u;
    }
    const uint32_t lds_k = lds_addr(&kbuf[0][0]) + (uint32_t)w * 8 * RBK;
    const uint32_t lds_v = lds_addr(&vbuf[0][0]) + (uint32_t)w * 8 * RBV;
    const int nkb_s = (p.S + F3_BK - 1) / F3_BK;   // key blocks holding keys < S
    const int nkb = CAUSAL ? min((qb * F3_BQ + F3_BQ) / F3_BK, nkb_s) : nkb_s;
    // block j -> stage j % F3_STAGES; blocks past the end re-read the last one so
    // that every MFMA phase issues the same number of DMAs (the vmcnt accounting).
    // A row at or past S gets an offset beyond the resource (2^31 > S * row bytes,
    // no wrap with soffset), so it reads zero whether or not the range check counts
    // soffset; its scores are masked.
    // (ntag: DMA instructions per tile; ctag: chunks per row, so 64 / CH rows per instruction)
    auto issue = [&](auto ntag, auto ctag, const v4i& rsrc, const uint32_t* voff, uint32_t lds, int tile, int j) {
        constexpr int DPT = decltype(ntag)::value, CH = decltype(ctag)::value;
        const int src = j < nkb ? j : nkb - 1;
        const uint32_t soff = (uint32_t)src * F3_BK * row_bytes;
        const uint32_t dst = lds + (uint32_t)(j % F3_STAGES) * tile;
        uint32_t v[DPT];
#pragma unroll
        for (int i = 0; i < DPT; ++i) v[i] = voff[i];
        if ((src + 1) * F3_BK > p.S) {   // uniform: only the ragged last block checks rows
#pragma unroll
            for (int i = 0; i < DPT; ++i)
                v[i] = src * F3_BK + 8 * w + (64 / CH) * i + lane / CH < p.S ? v[i] : 0x80000000u;
        }
#pragma unroll
        for (int i = 0; i < DPT; ++i) dma16(rsrc, v[i], soff, dst + 1024 * i);
    };
    auto issue_k = [&](int j) {
        issue(std::integral_constant<int, DPTK>{}, std::integral_constant<int, CHK>{}, rk, voff_k, lds_k, TILEK, j);
    };
    auto issue_v = [&](int j) {
        issue(std::integral_constant<int, DPTV>{}, std::integral_constant<int, CHV>{}, rv, voff_v, lds_v, TILEV, j);
    };
    constexpr int DPP = DPTK + DPTV;   // DMA instructions per wavefront and MFMA phase

    // K fragment (kt, ks): row 32 kt + r32, logical chunk 2 ks + h, stored at chunk ^ kswz(row)
    // (kswz depends on row % 16 = r32 % 16 only)
    // (2 ks + h) ^ kswz = 2 ks ^ (h ^ kswz) with kswz < 16 and the row's byte offset a multiple of
    // 32 chunks, so k_off[ks] = k_off[0] ^ 32 ks; at DQK = 256 that XOR is done per read instead of
    // holding 16 offsets in registers
    constexpr bool K_XOR = NKS > 8;
    int k_off[K_XOR ? 1 : NKS];
#pragma unroll
    for (int ks = 0; ks < (K_XOR ? 1 : NKS); ++ks) k_off[ks] = r32 * RBK + (((2 * ks + h) ^ kswz(r32)) << 4);
    auto k_ofs = [&](int ks) { return K_XOR ? (k_off[0] ^ (32 * ks)) : k_off[ks]; };
    // V^T fragment (dt, kk = 32 kt + 16 ks, read t = 0/1): source lane jj = (lane % 16) / 4,
    // q = lane % 4, dh = (lane / 16) % 2 addresses V[kk + 8 t + 4 h + jj][32 dt + 16 dh + 4 q],
    // logical chunk 4 dt + 2 dh + q / 2 stored at chunk ^ vswz(jj) (jj = key % 4 as kk % 8 == 0).
    int v_off[NDT];
    {
        const int jj = (lane & 15) >> 2, q = lane & 3, dh = (lane >> 4) & 1;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            v_off[dt] = (4 * h + jj) * RBV + (((4 * dt + 2 * dh + (q >> 1)) ^ vswz(jj)) << 4) + ((q & 1) << 3);
    }

    f32x16 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m_run = -INFINITY;   // running max of the scaled scores (log2 units)
    float l_run = 0.f;         // this lane's partial row sum
    const float c = p.scale_log2;
    f32x16 st[2];              // S^T of the current block: st[kt] register r = key 32 kt + 8 (r / 4) + 4 h + r % 4
    f16x8 pf[2][2];            // P^T of the previous block, B operand [kt][ks]: keys 32 kt + 16 ks + 8 (i / 4) + 4 h + i % 4

    // The MFMA phase as one list of NOPS operations -- ops [0, NPV): O^T += V^T P^T
    // for the previous block (kt = i / (2 NDT), ks = i / NDT % 2, dt = i % NDT); ops
    // [NPV, NOPS): S^T = K Q^T (ks = (i - NPV) / 2, kt = i % 2) -- whose LDS operand
    // reads run PREF operations ahead of the MFMAs (the partner wavefront is in
    // its softmax phase, so nothing else hides the LDS latency).
    auto read_op = [&](int i, const uint8_t* vbase, const uint8_t* kbase) -> f16x8 {
        if (i < NPV) {
            const int kk = 32 * (i / (2 * NDT)) + 16 * ((i / NDT) & 1), dt = i % NDT;
            const f3_s16x4 lo = f3_read_tr(vbase + v_off[dt] + kk * RBV);
            const f3_s16x4 hi = f3_read_tr(vbase + v_off[dt] + (kk + 8) * RBV);
            return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
        const int j = i - NPV;
        return *reinterpret_cast<const f16x8*>(kbase + k_ofs(j >> 1) + (j & 1) * 32 * RBK);
    };
    auto mma_op = [&](int i, f16x8 a) {
        if (i < NPV) {
            o[i % NDT] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[i / (2 * NDT)][(i / NDT) & 1], o[i % NDT], 0,
                                                                 0, 0);
        } else {
            const int j = i - NPV;
            st[j & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[j >> 1], j < 2 ? f32x16{} : st[j & 1], 0, 0, 0);
        }
    };
    auto mfma_phase = [&](auto pv_tag, auto s_tag, const uint8_t* vbase, const uint8_t* kbase) {
        constexpr int first = decltype(pv_tag)::value ? 0 : NPV;
        constexpr int last = decltype(s_tag)::value ? NOPS : NPV;
        f16x8 buf[PREF];
#pragma unroll
        for (int t = 0; t < PREF; ++t)
            if (first + t < last) buf[t] = read_op(first + t, vbase, kbase);
#pragma unroll
        for (int i = first; i < last; ++i) {
            const f16x8 a = buf[(i - first) % PREF];
            if (i + PREF < last) buf[(i - first) % PREF] = read_op(i + PREF, vbase, kbase);
            mma_op(i, a);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (decltype(s_tag)::value) {
            f3_pin(st[0]);
            f3_pin(st[1]);
        }
    };

    issue_k(0);
    // Consume Q here so the compiler's own wait for its loads happens once, before
    // the loop, instead of as vmcnt waits inside it (which would also cover the
    // DMAs issued in the loop, since it does not count those).
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        const uint4 u = __builtin_bit_cast(uint4, qf[ks]);
        asm volatile("" ::"v"(u.x), "v"(u.y), "v"(u.z), "v"(u.w));
    }
    issue_k(1);
    issue_v(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (late) __builtin_amdgcn_s_barrier();

    // Online softmax of block kb (base 2, the scale folded into the exponent's fma):
    // masks the diagonal block, rescales O and L when the maximum moves (lazily),
    // and leaves P^T in pf for the next MFMA phase.
    auto softmax = [&](int kb) {
        const int key0 = kb * F3_BK;
        if (CAUSAL && key0 + F3_BK - 1 > q0) {
            // (for a query < S every key past S is also past the query)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * h + (r & 3);
                    st[kt][r] = key > my_q ? -INFINITY : st[kt][r];
                }
        } else if (!CAUSAL && key0 + F3_BK > p.S) {   // the ragged last key block
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * h + (r & 3);
                    st[kt][r] = key >= p.S ? -INFINITY : st[kt][r];
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[kt][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
        if (__builtin_amdgcn_ballot_w64(mx > m_run + F3_RESCALE)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            m_run = m_new;
        }
        const float mneg = -m_run;
        float lsum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                f16x8 pv;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float e = __builtin_amdgcn_exp2f(fmaf(st[kt][8 * ks + i], c, mneg));
                    lsum += e;
                    pv[i] = (f16)e;
                }
                pf[kt][ks] = pv;
            }
        l_run += lsum;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) f3_pin(pf[kt][ks]);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) f3_pin(o[dt]);
        asm volatile("; pin" ::"v"(l_run), "v"(m_run));
    };
    // Every MFMA phase issues the DMAs of K block kb + 2 and V block kb + 1: the
    // tiles are loaded cooperatively, so each wavefront issues its share of every
    // one, active or not, and passes the same barriers.
    auto dma = [&](int kb) {
        issue_k(kb + 2);
        issue_v(kb + 1);
    };
    auto vb = [&](int kb) { return &vbuf[(kb + F3_STAGES - 1) % F3_STAGES][0]; };   // V of block kb - 1
    auto kbuf_of = [&](int kb) { return &kbuf[kb % F3_STAGES][0]; };
    // this wavefront's last block with an unmasked key
    const int last = CAUSAL ? min(nkb - 1, (q0 + 31) / F3_BK) : nkb - 1;

    // iteration 0: S only
    dma(0);
    mfma_phase(f3_tag<false>{}, f3_tag<true>{}, vb(0), kbuf_of(0));
    f3_phase_end<DPP>();
    softmax(0);
    f3_phase_end<DPP>();
    // iterations 1 .. last: O += V^T P^T for block kb - 1, then S for block kb
    for (int kb = 1; kb <= last; ++kb) {
        dma(kb);
        mfma_phase(f3_tag<true>{}, f3_tag<true>{}, vb(kb), kbuf_of(kb));
        f3_phase_end<DPP>();
        softmax(kb);
        f3_phase_end<DPP>();
    }
    // iteration last + 1: the final O update
    dma(last + 1);
    mfma_phase(f3_tag<true>{}, f3_tag<false>{}, vb(last + 1), kbuf_of(last + 1));
    f3_phase_end<DPP>();
    f3_phase_end<DPP>();
    // remaining iterations (causal: blocks past this wavefront's queries)
    for (int kb = last + 2; kb <= nkb; ++kb) {
        dma(kb);
        f3_phase_end<DPP>();
        f3_phase_end<DPP>();
    }
    if (!late) __builtin_amdgcn_s_barrier();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- O / L, fp16.  o[dt] register r: d = 32 dt + 8 (r / 4) + 4 h + r % 4 of query my_q.
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.f / l_tot;
    if (my_q >= p.S) return;
    f16* orow = Ob + (int64_t)my_q * p.osl;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = 32 * dt + 8 * g4 + 4 * h;
            f16x4 v = {(f16)(o[dt][4 * g4 + 0] * inv), (f16)(o[dt][4 * g4 + 1] * inv),
                       (f16)(o[dt][4 * g4 + 2] * inv), (f16)(o[dt][4 * g4 + 3] * inv)};
            if (DQK != 256 || d < p.dv) __builtin_nontemporal_store(v, reinterpret_cast<f16x4*>(orow + d));
        }
}

// ---- flash_fwd5_kernel: score and output wavefronts ----
//
// Same transposed formulation (S^T = K Q^T, O^T = V^T P^T on 32x32x16 f16 MFMAs, a
// lane owns one query per 32-query half), with the work of 64 queries split between
// the two wavefronts that share a SIMD (w and w + 4):
//  * score wavefront w (0-3): Q^T of its 64 queries in registers; per key block it
//    computes S^T = K Q^T (32 MFMAs), the online softmax (lazy rescale), and writes
//    P^T as MFMA B-operand fragments (8 KB) and the rescale factors to workgroup
//    memory;
//  * output wavefront w + 4: O^T of the same 64 queries in registers; per key block
//    it rescales O when told to and adds V^T P^T (32 MFMAs).
// Every K or V fragment read from LDS feeds two MFMAs (two 32-query halves), and the
// score wavefront's softmax VALU runs beside the output wavefront's MFMAs on the same
// SIMD -- no phase barrier between them, one workgroup barrier per key block.
// Score wavefronts compute S for block j + 1 while output wavefronts add P V of block
// j; P is double-buffered.  One workgroup = 8 wavefronts = 256 queries; K in a
// three-stage LDS ring, V in two stages.  The output wavefronts, which wait for the
// score wavefronts, also issue every K and V load and sum the rows of P (from the
// fp16 fragments they read, in fp32) -- the score wavefront does only the scores and
// the softmax.
constexpr int F5_PAIRS = 4;
constexpr int F5_BQ = 64 * F5_PAIRS;   // 256 queries per workgroup
constexpr int F5_BK = 64;
constexpr int F5_KST = 3, F5_VST = 2;
constexpr int F5_PFK = 4;              // K fragments read ahead of the MFMA that uses them
constexpr int F5_PFV = 5;              // V fragments read ahead

typedef _Float16 f5_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t f5_u32x4 __attribute__((ext_vector_type(4)));

// x in lanes 0-31 and 32-63 as two registers: one v_permlane32_swap between two
// distinct copies of x (the builtin with one value twice may be given one register,
// and a register swapped with itself does not produce both halves)
__device__ __forceinline__ void f5_xor32_pair(float x, float& a, float& b) {
    a = x;
    b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// q = fp16(q * c) in place, two elements per instruction: the mixed-precision FMA takes an fp16
// half of q (op_sel picks which), fp32 c and a zero addend, and rounds the exact product once to
// fp16 (measured over all 65536 fp16 values at four scales: the correctly rounded product in every
// case, except that -0 comes out +0, which adds nothing to a dot product; (f16)((float)q * c),
// rounded twice, differs in up to 3 % of them) -- one instruction instead of two converts, a
// multiply and a pack.  The trailing s_nop gives a following MFMA that reads q the wait states a
// VALU write needs before it (this is asm, so the compiler does not count it as a VALU write).
__device__ __forceinline__ void fa_scale_f16(f16x8& q, float c) {
    uint4 u = __builtin_bit_cast(uint4, q);
    asm("v_fma_mixlo_f16 %0, %0, %4, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %0, %4, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %1, %1, %4, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %1, %1, %4, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %2, %2, %4, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %2, %2, %4, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixlo_f16 %3, %3, %4, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %3, %3, %4, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "s_nop 1"
        : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w)
        : "v"(c));
    q = __builtin_bit_cast(f16x8, u);
}

// DE: the head dimension the MFMAs cover, 64, 96 or 128 (D rounded up to a multiple of 32).  K, V
// and Q are staged 128 wide whatever DE is (the chunks past D are DMA-ed as zeros, so the LDS
// layout, its swizzles and the DMA map stay those of D = 128); a smaller DE only drops the S^T
// k-steps and the O^T row tiles that would multiply those zero columns.
template <bool CAUSAL, int DE>
__global__ void __launch_bounds__(128 * F5_PAIRS, 1) flash_fwd5_kernel(FaParams p) {
    static_assert(DE == 64 || DE == 96 || DE == 128, "the MFMAs cover 64, 96 or 128 of the head dimension");
    constexpr int DH = 128;                    // staged width
    constexpr int RB = DH * 2;                 // 256 bytes per K / V row
    constexpr int CH = RB / 16;                // 16 chunks
    constexpr int TILE = F5_BK * RB;           // 16 KB
    constexpr int NKS = DE / 16;               // k-steps of S^T (8 at DE = 128)
    constexpr int NDT = DE / 32;               // O^T row tiles (4 at DE = 128)
    constexpr int NSF = 2 * NKS;               // K fragments per block: (ks, kt)
    constexpr int NVF = 4 * NDT;               // V fragments per block: (key step kk, dt)
    constexpr int DPT = TILE / (1024 * F5_PAIRS);   // 4 DMA instructions per wavefront per tile
    constexpr int PBUF = 8 * 1024;             // one pair's P^T fragments for one block
    static_assert(DPT == 4, "4 DMA instructions per tile and wavefront");
    __shared__ __attribute__((aligned(1024))) uint8_t kbuf[F5_KST][TILE];   // [key][RB], chunk ^ key % 16
    __shared__ __attribute__((aligned(1024))) uint8_t vbuf[F5_VST][TILE];   // [key][RB], chunk ^ 4 (key % 4)
    __shared__ __attribute__((aligned(1024))) uint8_t pbuf[2][F5_PAIRS][PBUF];
    __shared__ float abuf[2][F5_PAIRS][64];    // rescale factor per query of the next block
    __shared__ int fbuf[2][F5_PAIRS];          // whether that block rescales

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool is_s = w < F5_PAIRS;
    const int pr = w & (F5_PAIRS - 1);         // the pair: queries q0 .. q0 + 63
    const int nqb = (p.S + F5_BQ - 1) / F5_BQ;
    const int nbh = p.H * p.B;
    int bh, qb;
    fa_order(nqb, nbh, CAUSAL, bh, qb);
    const int hh = bh % p.H, bb = bh / p.H;
    const int64_t head = (int64_t)hh * p.sh + (int64_t)bb * p.sb;
    f16* Ob = p.O + (int64_t)hh * p.osh + (int64_t)bb * p.osb;
    const int q0 = qb * F5_BQ + pr * 64;
    const int r32 = lane & 31, h = lane >> 5;
    const int nkb_s = (p.S + F5_BK - 1) / F5_BK;
    const int nkb = CAUSAL ? min((qb + 1) * (F5_BQ / F5_BK), nkb_s) : nkb_s;
    const int last = CAUSAL ? min(nkb - 1, (q0 + 63) / F5_BK) : nkb - 1;   // this pair's last key block

    // LDS-DMA of K and V (issued by the output wavefronts): wavefront pr moves rows
    // 16 pr + 4 i + lane / 16 of a tile, physical chunk lane % 16 (K chunk ^ key % 16, V
    // chunk ^ 4 (key % 4)).  The lane offsets are the same for every block; the buffer
    // resource of a block starts at its first row and ends at the sequence's end, so rows
    // at or past S read zero.  Blocks past the end re-read the last one (every iteration
    // issues the same DMAs).
    // A head dimension D < 128 (a multiple of 8) runs zero-padded to 128: a lane whose logical
    // chunk lies at or past D / 8 takes an offset beyond every buffer resource's range, so its
    // DMA writes zero into LDS -- zero Q and K columns add nothing to the scores, and the O
    // columns that the zero V columns produce are not stored.
    const uint32_t row_bytes = (uint32_t)(p.sl * 2);
    const int dch = p.D >> 3;                  // 16-byte chunks of a row that hold data
    auto chunk_ofs = [&](int row, int c) -> uint32_t {
        return c < dch ? (uint32_t)row * row_bytes + 16u * (uint32_t)c : 0x80000000u;
    };
    uint32_t dv_k[DPT], dv_v[DPT];
#pragma unroll
    for (int i = 0; i < DPT; ++i) {
        const int row = 16 * pr + 4 * i + lane / CH;
        dv_k[i] = chunk_ofs(row, (lane % CH) ^ (row & 15));
        dv_v[i] = chunk_ofs(row, (lane % CH) ^ (4 * (row & 3)));
    }
    auto dma_tile = [&](bool is_k, int j) __attribute__((always_inline)) {
        const int src = j < nkb ? j : nkb - 1;
        const f16* base = (is_k ? p.K : p.V) + head + (int64_t)src * F5_BK * p.sl;
        const uint32_t rows = (uint32_t)min(F5_BK, p.S - src * F5_BK);
        const v4i rs = make_rsrc(base, rows * row_bytes);
        const uint32_t dst = lds_addr(is_k ? &kbuf[0][0] : &vbuf[0][0]) + (uint32_t)pr * 16 * RB +
                             (uint32_t)(j % (is_k ? F5_KST : F5_VST)) * TILE;
#pragma unroll
        for (int i = 0; i < DPT; ++i)
            dma16(rs, is_k ? dv_k[i] : dv_v[i], 0u, __builtin_amdgcn_readfirstlane(dst + 1024u * i));
    };
    typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
    typedef __attribute__((address_space(3))) f3_s16x4 lds_s16x4;
    // P^T fragment (kt, ks, qh) of pair pr in buffer b: 1 KB, lane l at 16 l
    const uint32_t p_lane = lds_addr(&pbuf[0][0][0]) + (uint32_t)pr * PBUF + 16u * lane;
    auto paddr = [&](int b, int kt, int ks, int qh) __attribute__((always_inline)) -> uint32_t {
        return p_lane + (uint32_t)(b * F5_PAIRS * PBUF + ((kt * 2 + ks) * 2 + qh) * 1024);
    };

    // prologue DMAs (output wavefronts): K_0, K_1, K_2, V_0
    if (!is_s) {
#pragma unroll
        for (int t = 0; t < 3; ++t) dma_tile(true, t);
        dma_tile(false, 0);
    }

    if (is_s) {
        // ================= score wavefront =================
        // The pair's 64 Q rows go to LDS first (this pair's P buffers, free until the first
        // block's P is written), in the K tile's layout -- LDS-DMA of 4 whole rows per
        // instruction, chunk ^ row % 16, rows at or past S read zero -- and the Q^T
        // fragments are read from there: whole-row reads instead of 32 rows x 32 bytes per
        // load instruction.
        const uint32_t qst[2] = {lds_addr(&pbuf[0][pr][0]), lds_addr(&pbuf[1][pr][0])};
        {
            const uint32_t rows = (uint32_t)max(0, min(64, p.S - q0));
            const v4i rs = make_rsrc(p.Q + head + (int64_t)q0 * p.sl, rows * row_bytes);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = 4 * i + lane / CH;
                const uint32_t v = chunk_ofs(row, (lane % CH) ^ (row & 15));
                dma16(rs, v, 0u, __builtin_amdgcn_readfirstlane(qst[i / 8] + (uint32_t)((4 * i) % 32) * RB));
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        f16x8 qf[2][NKS];   // Q^T B operands: query q0 + 32 qh + r32, d = 16 ks + 8 h + [0, 8)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
                qf[qh][ks] = *(const lds_f16x8*)(uintptr_t)(qst[qh] + (uint32_t)(r32 * RB + (((2 * ks + h) ^ (r32 & 15)) << 4)));
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const uint4 u = __builtin_bit_cast(uint4, qf[qh][ks]);
                asm volatile("" ::"v"(u.x), "v"(u.y), "v"(u.z), "v"(u.w));
            }
        // The base-2 softmax scale c is folded into Q^T (one fp16 rounding of q * c) when
        // that cannot overflow (c <= 1), and the running maximum enters the product as a
        // bias k-step: ones (key rows, k = 0) times -m (query columns, k = 0).  The
        // accumulator then holds S' = c q.k - m directly and P = exp2(S') needs no
        // per-score multiply-add.  m is kept fp16-representable for that; a rescaled block,
        // c > 1, or a maximum beyond +-60000 (after which the wavefront stays on this path)
        // take P = exp2(fma(S, c', -m')) in fp32 instead.
        const float c = p.scale_log2;
        bool fast = c <= 1.f;                    // wavefront-uniform
        if (fast) {
#pragma unroll
            for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) fa_scale_f16(qf[qh][ks], c);
        }
        const float c_raw = fast ? 1.f : c;      // the multiplier S needs on the fp32 path
        f16x8 ones{};                            // bias A operand: 1 at k = 0 of every key row
        ones[0] = h == 0 ? (f16)1.f : (f16)0.f;
        f16x8 qm[2] = {f16x8{}, f16x8{}};         // bias B operand: -m at k = 0 of each query
        // K fragment (kt, ks): row 32 kt + r32, chunk (2 ks + h) ^ (r32 % 16)
        uint32_t kb0[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
            kb0[ks] = lds_addr(&kbuf[0][0]) + (uint32_t)(r32 * RB + (((2 * ks + h) ^ (r32 & 15)) << 4));
        f32x16 st[2][2];           // st[kt][qh] register r: key 32 kt + 8 (r / 4) + 4 h + r % 4
        float m_run[2] = {0.f, 0.f};

        // S_kb = K_kb Q^T (minus m), the softmax, P^T and the rescale factors into buffer b
        auto block = [&](int kb, int b, bool first) __attribute__((always_inline)) {
            uint32_t ka[NKS];
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                ka[ks] = kb0[ks] + (uint32_t)((kb % F5_KST) * TILE);
                asm("; lds address" : "+v"(ka[ks]));
            }
            auto kread = [&](int f) __attribute__((always_inline)) -> f16x8 {   // f = 2 ks + kt
                return *(const lds_f16x8*)(uintptr_t)(ka[f >> 1] + (uint32_t)((f & 1) * 32 * RB));
            };
            // reads F5_PFK fragments ahead of their MFMAs; sched_barrier keeps this order
            // (the scheduler otherwise moves each read next to its use)
            f16x8 fr[F5_PFK];
#pragma unroll
            for (int f = 0; f < F5_PFK; ++f) fr[f] = kread(f);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int qh = 0; qh < 2; ++qh)
                    st[kt][qh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, qm[qh], f32x16{}, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 2 * NSF; ++i) {   // MFMA i: fragment f = i / 2 (ks = f / 2, kt = f % 2), qh = i % 2
                const int f = i >> 1, qh = i & 1, ks = f >> 1, kt = f & 1;
                st[kt][qh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[f % F5_PFK], qf[qh][ks], st[kt][qh], 0, 0, 0);
                if (qh == 1 && f + F5_PFK < NSF) fr[f % F5_PFK] = kread(f + F5_PFK);
                __builtin_amdgcn_sched_barrier(0);
            }
            // mask: causal key > query; else keys >= S.  A pair's causal last block is its diagonal
            // block (it starts at the pair's first query, kb * 64 = q0, for every pair with a query
            // below S; the others are never stored), where key tile 1 lies wholly above query half
            // 0 and key tile 0 wholly below query half 1: only the two diagonal 32 x 32 tiles compare.
            if (CAUSAL ? kb == last : (kb + 1) * F5_BK > p.S) {
                int dv = CAUSAL ? 4 * h - r32 : kb * F5_BK + 4 * h - p.S;
                asm volatile("; mask" : "+v"(dv));
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int kr = 32 * kt + 8 * (r >> 2) + (r & 3);
                            if (CAUSAL && kt != qh) {
                                if (kt > qh) st[kt][qh][r] = -INFINITY;
                                continue;
                            }
                            const bool off = CAUSAL ? dv > 32 * qh - kr : dv >= -kr;
                            st[kt][qh][r] = off ? -INFINITY : st[kt][qh][r];
                        }
            }
            // t = how far this block's largest exponent lies above the running maximum
            const bool fast_blk = fast;           // st holds S' (fast) or S (fp32 path)
            float vl[2];   // this lane's largest score per query half
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
                float v = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) v = fmaxf(v, st[kt][qh][r]);
                vl[qh] = fast_blk ? v : fmaf(v, c_raw, -m_run[qh]);
            }
            const bool rescale = first || __builtin_amdgcn_ballot_w64(vl[0] > F3_RESCALE || vl[1] > F3_RESCALE) != 0;
            float sub[2] = {0.f, 0.f};
            if (rescale) {
                float t[2];
#pragma unroll
                for (int qh = 0; qh < 2; ++qh) {
                    float a, bb2;
                    f5_xor32_pair(vl[qh], a, bb2);
                    t[qh] = fmaxf(a, bb2);
                }
                float mn[2];
                bool ovf = false;
#pragma unroll
                for (int qh = 0; qh < 2; ++qh) {
                    // the first block sets m to its maximum (it always holds key 0, so it
                    // is never fully masked); later ones only raise it
                    mn[qh] = m_run[qh] + (first ? t[qh] : fmaxf(t[qh], 0.f));
                    ovf = ovf || !(fabsf(mn[qh]) <= 60000.f);
                }
                if (fast && __builtin_amdgcn_ballot_w64(ovf) != 0) fast = false;
                float alpha[2];
#pragma unroll
                for (int qh = 0; qh < 2; ++qh) {
                    if (fast) mn[qh] = (float)(f16)mn[qh];
                    alpha[qh] = __builtin_amdgcn_exp2f(m_run[qh] - mn[qh]);
                    sub[qh] = fast_blk ? mn[qh] - m_run[qh] : mn[qh];
                    m_run[qh] = mn[qh];
                    qm[qh][0] = (fast && h == 0) ? (f16)(-mn[qh]) : (f16)0.f;
                }
                if (h == 0) {
                    abuf[b][pr][r32] = alpha[0];
                    abuf[b][pr][32 + r32] = alpha[1];
                }
            } else if (!fast_blk) {
                sub[0] = m_run[0];
                sub[1] = m_run[1];
            }
            if (lane == 0) fbuf[b][pr] = rescale ? 1 : 0;
            // P = exp2(S') (or exp2(S c' - m')) in fp16 (RNE), stored as the output wavefront's B operands
            auto pstore = [&](auto plain) __attribute__((always_inline)) {
                const float cb = fast_blk ? 1.f : c_raw;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int qh = 0; qh < 2; ++qh) {
                            f5_u32x4 u;
                            const float msub = -sub[qh];
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const int r0 = 8 * ks + 2 * k;
                                float x0 = st[kt][qh][r0], x1 = st[kt][qh][r0 + 1];
                                if constexpr (!decltype(plain)::value) {
                                    x0 = fmaf(x0, cb, msub);
                                    x1 = fmaf(x1, cb, msub);
                                }
                                const f5_h2 hv = {(_Float16)__builtin_amdgcn_exp2f(x0), (_Float16)__builtin_amdgcn_exp2f(x1)};
                                u[k] = __builtin_bit_cast(uint32_t, hv);
                            }
                            *(__attribute__((address_space(3))) f5_u32x4*)(uintptr_t)paddr(b, kt, ks, qh) = u;
                        }
            };
            if (fast_blk && !rescale)
                pstore(f3_tag<true>{});
            else
                pstore(f3_tag<false>{});
        };

        __syncthreads();                         // K_0 .. K_2, V_0 in LDS
        block(0, 0, true);
        __syncthreads();                         // P_0 published
        for (int j = 0; j < nkb; ++j) {
            if (j + 1 <= last) block(j + 1, (j + 1) & 1, false);
            __syncthreads();
        }
    } else {
        // ================= output wavefront =================
        // V^T fragment (dt, kk): two transposing reads at keys kk + 4 h + jj and + 8
        uint32_t vb0[NDT];
        {
            const int jj = (lane & 15) >> 2, q = lane & 3, dh = (lane >> 4) & 1;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                vb0[dt] = lds_addr(&vbuf[0][0]) +
                          (uint32_t)((4 * h + jj) * RB + (((4 * dt + 2 * dh + (q >> 1)) ^ (4 * jj)) << 4) + ((q & 1) << 3));
        }
        f32x16 o[NDT][2];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][qh][r] = 0.f;
        float l_run[2] = {0.f, 0.f};             // this lane's partial row sums of P
        const f5_h2 ones = {(_Float16)1.f, (_Float16)1.f};

        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();                         // K_0 .. K_2, V_0 in LDS
        __syncthreads();                         // P_0 published
        for (int j = 0; j < nkb; ++j) {
            const int b = j & 1;
            // K_{j+3} into K_j's stage and V_{j+1} into V_{j-1}'s (both read in iteration j - 1)
            dma_tile(true, j + 3);
            dma_tile(false, j + 1);
            if (j <= last) {
                if (j > 0 && fbuf[b][pr] != 0) {   // the maximum moved at block j: O *= alpha
                    const float a0 = abuf[b][pr][r32], a1 = abuf[b][pr][32 + r32];
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            o[dt][0][r] *= a0;
                            o[dt][1][r] *= a1;
                        }
                    l_run[0] *= a0;
                    l_run[1] *= a1;
                }
                uint32_t va[NDT];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    va[dt] = vb0[dt] + (uint32_t)((j % F5_VST) * TILE);
                    asm("; lds address" : "+v"(va[dt]));
                }
                auto vread = [&](int f) __attribute__((always_inline)) -> f16x8 {   // f = NDT kk + dt
                    const int kk = 16 * (f / NDT), dt = f % NDT;
                    const f3_s16x4 lo =
                        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(va[dt] + (uint32_t)(kk * RB)));
                    const f3_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(uintptr_t)(va[dt] + (uint32_t)((kk + 8) * RB)));
                    return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                };
                auto pread = [&](int kk, int qh) __attribute__((always_inline)) -> f16x8 {
                    return *(const lds_f16x8*)(uintptr_t)paddr(b, kk >> 1, kk & 1, qh);
                };
                // V fragments F5_PFV ahead, P one key step ahead; sched_barrier keeps the order
                f16x8 fr[F5_PFV];
                f16x8 pp[2][2];   // [kk % 2][qh]
                pp[0][0] = pread(0, 0);
                pp[0][1] = pread(0, 1);
#pragma unroll
                for (int f = 0; f < F5_PFV; ++f) fr[f] = vread(f);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 2 * NVF; ++i) {   // MFMA i: V fragment f = i / 2 (kk = f / NDT, dt = f % NDT), qh = i % 2
                    const int f = i >> 1, qh = i & 1, kk = f / NDT, dt = f % NDT;
                    if (i % (2 * NDT) == 0 && kk < 3) {   // the next key step's P fragments
                        pp[(kk + 1) & 1][0] = pread(kk + 1, 0);
                        pp[(kk + 1) & 1][1] = pread(kk + 1, 1);
                    }
                    if (i % (2 * NDT) == NDT) {   // row sums of this key step's P (fp16 values, fp32 sum)
#pragma unroll
                        for (int qq = 0; qq < 2; ++qq)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                l_run[qq] = __builtin_amdgcn_fdot2(f5_h2{pp[kk & 1][qq][2 * e], pp[kk & 1][qq][2 * e + 1]},
                                                                   ones, l_run[qq], false);
                    }
                    o[dt][qh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[f % F5_PFV], pp[kk & 1][qh], o[dt][qh], 0, 0,
                                                                       0);
                    if (qh == 1 && f + F5_PFV < NVF) fr[f % F5_PFV] = vread(f + F5_PFV);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // K_{j+3}, V_{j+1} landed
            __syncthreads();
        }
        // ---- O / L, fp16.  o[dt][qh] register r: d = 32 dt + 8 (r / 4) + 4 h + r % 4 of query q0 + 32 qh + r32.
        float inv[2];
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
            float la, lb;
            f5_xor32_pair(l_run[qh], la, lb);
            inv[qh] = 1.f / (la + lb);
        }
        if (p.o16) {
            // Staged through this pair's P buffers (no wavefront reads them after the last
            // barrier) as 64 rows of 256 bytes, chunk ^ row % 16, then stored 4 whole rows per
            // instruction (16 bytes per lane) instead of 32 rows x 16 bytes.
            const uint32_t ost[2] = {lds_addr(&pbuf[0][pr][0]), lds_addr(&pbuf[1][pr][0])};
            typedef __attribute__((address_space(3))) f16x4 lds_f16x4;
#pragma unroll
            for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        const f16x4 v = {(f16)(o[dt][qh][4 * g4 + 0] * inv[qh]), (f16)(o[dt][qh][4 * g4 + 1] * inv[qh]),
                                         (f16)(o[dt][qh][4 * g4 + 2] * inv[qh]), (f16)(o[dt][qh][4 * g4 + 3] * inv[qh])};
                        *(lds_f16x4*)(uintptr_t)(ost[qh] + (uint32_t)(r32 * RB + (((4 * dt + g4) ^ (r32 & 15)) << 4) + 8 * h)) = v;
                    }
            // all 16 rows of a lane group read before the first store (one LDS round trip), one
            // 64-bit base per lane and a row stride
            const int lrow = lane / CH, cc = lane % CH;
            f16x8 rv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = 4 * i + lrow;
                rv[i] = *(const lds_f16x8*)(uintptr_t)(ost[i / 8] + (uint32_t)((row % 32) * RB + ((cc ^ (row & 15)) << 4)));
            }
            f16* obase = Ob + (int64_t)(q0 + lrow) * p.osl + 8 * cc;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (q0 + 4 * i + lrow < p.S && cc < dch)
                    __builtin_nontemporal_store(rv[i], reinterpret_cast<f16x8*>(obase + (int64_t)(4 * i) * p.osl));
        } else {
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
                const int q = q0 + 32 * qh + r32;
                if (q >= p.S) continue;
                f16* orow = Ob + (int64_t)q * p.osl;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        const int d = 32 * dt + 8 * g4 + 4 * h;
                        f16x4 v = {(f16)(o[dt][qh][4 * g4 + 0] * inv[qh]), (f16)(o[dt][qh][4 * g4 + 1] * inv[qh]),
                                   (f16)(o[dt][qh][4 * g4 + 2] * inv[qh]), (f16)(o[dt][qh][4 * g4 + 3] * inv[qh])};
                        if (d < p.D) __builtin_nontemporal_store(v, reinterpret_cast<f16x4*>(orow + d));
                    }
            }
        }
    }
}

// Any D <= 256, any S: one thread per query row, online softmax in fp32 over every
// key (the clamped/ragged path; not the fast one).
__global__ void flash_generic_kernel(FaParams p, int D) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)p.S * p.H * p.B;
    if (t >= total) return;
    const int qrow = (int)(t % p.S);
    const int64_t bh = t / p.S;
    const int h = (int)(bh % p.H), b = (int)(bh / p.H);
    const f16* q = p.Q + h * p.sh + b * p.sb + (int64_t)qrow * p.sl;
    const f16* Kb = p.K + h * p.sh + b * p.sb;
    const f16* Vb = p.V + h * p.sh + b * p.sb;
    float acc[256];
    for (int e = 0; e < D; ++e) acc[e] = 0.f;
    float m = -3.0e38f, l = 0.f;
    const int nk = p.causal ? qrow + 1 : p.S;
    for (int j = 0; j < nk; ++j) {
        const f16* k = Kb + (int64_t)j * p.sl;
        float s = 0.f;
        for (int e = 0; e < D; ++e) s = fmaf((float)q[e], (float)k[e], s);
        s *= p.scale_log2;
        const float mn = fmaxf(m, s);
        const float a = exp2f(m - mn), e1 = exp2f(s - mn);
        const f16* v = Vb + (int64_t)j * p.sl;
        for (int e = 0; e < D; ++e) acc[e] = acc[e] * a + e1 * (float)v[e];
        l = l * a + e1;
        m = mn;
    }
    f16* o = p.O + h * p.osh + b * p.osb + (int64_t)qrow * p.osl;
    for (int e = 0; e < D; ++e) o[e] = (f16)(acc[e] / l);
}

}  // namespace lava

using namespace lava;

extern "C" int lava_hip_flash_attn_fwd_f16(const void* Q, const void* K, const void* V, void* O, int64_t B, int64_t H,
                                           int64_t S, int64_t D, const int64_t* strides, const int64_t* ostrides,
                                           float scale, int causal, void* stream) {
    LAVA_ARG(B >= 0 && H >= 0 && S >= 0 && D >= 0, "flash_attn_fwd_f16: negative extent");
    if (B == 0 || H == 0 || S == 0) return LAVA_HIP_OK;
    LAVA_ARG(D >= 1, "flash_attn_fwd_f16: D = 0 with S > 0");
    LAVA_ARG(Q && K && V && O && strides, "flash_attn_fwd_f16: null pointer");
    LAVA_ARG(scale == scale && scale != INFINITY && scale != -INFINITY, "flash_attn_fwd_f16: scale is not finite");
    const int64_t* os = ostrides ? ostrides : strides;
    LAVA_ARG(strides[0] == 1 && os[0] == 1, "flash_attn_fwd_f16: the head dimension (E) must be contiguous");
    for (int i = 1; i < 4; ++i)
        LAVA_ARG(strides[i] >= 0 && os[i] >= 0, "flash_attn_fwd_f16: negative stride %d", i);
    LAVA_ARG(strides[1] >= D && os[1] >= D, "flash_attn_fwd_f16: sequence stride smaller than D");
    LAVA_ARG(S <= 0x7fffffff && H <= 0x7fffffff && B <= 0x7fffffff, "flash_attn_fwd_f16: extent too large");
    LAVA_ARG(aligned(Q, 2) && aligned(K, 2) && aligned(V, 2) && aligned(O, 2), "flash_attn_fwd_f16: misaligned");
    LAVA_REQUIRE(D <= 256, LAVA_HIP_ERR_UNSUPPORTED, "flash_attn_fwd_f16: D = %lld > 256 is not supported",
                 (long long)D);
    int rc = lava_hip_init();
    if (rc != LAVA_HIP_OK) return rc;

    FaParams p;
    p.Q = (const f16*)Q;
    p.K = (const f16*)K;
    p.V = (const f16*)V;
    p.O = (f16*)O;
    p.sl = strides[1];
    p.sh = strides[2];
    p.sb = strides[3];
    p.osl = os[1];
    p.osh = os[2];
    p.osb = os[3];
    p.S = (int)S;
    p.H = (int)H;
    p.B = (int)B;
    p.scale_log2 = scale * 1.4426950408889634f;
    p.causal = causal != 0;
    p.o16 = aligned(O, 16) && os[1] % 8 == 0 && os[2] % 8 == 0 && os[3] % 8 == 0;
    p.D = (int)D;
    p.dv = (int)D;
    hipStream_t s = as_stream(stream);

    // D <= 128 (a multiple of 8) with 16-byte rows, and D = 256: the MFMA kernels.  D <= 128 runs
    // on flash_fwd5_kernel (score/output wavefront pairs, rows staged zero-padded to 128, MFMAs over
    // D rounded up to 64, 96 or 128; the scale folds into Q^T, so any sign; at D = 64 it runs
    // 1.2x flash_fwd3_kernel, 837 against 682 TFLOP/s causal at B=4 H=32 S=4096), D = 256 with a
    // positive scale on flash_fwd3_kernel (ping-pong wavefront pairs; its base-2 running maximum
    // assumes one); all take any S (a ragged last block of queries or keys is zero-filled and
    // masked).  lava_hip_set_kernel_override(LAVA_HIP_FAMILY_ATTN, 3) pins flash_fwd3_kernel for
    // D = 64 and 128 with a positive scale (tests and A/B timing).  Everything else runs on
    // flash_generic_kernel.
    bool lay_ok = D >= 8 && D <= FA_D && D % 8 == 0 && strides[0] == 1 && os[0] == 1;
    for (int i = 1; i < 4; ++i) lay_ok = lay_ok && strides[i] % 8 == 0 && os[i] % 4 == 0;
    lay_ok = lay_ok && aligned(Q, 16) && aligned(K, 16) && aligned(V, 16) && aligned(O, 8) &&
             S * strides[1] * 2 < ((int64_t)1 << 31);
    const int64_t blocks3 = ((S + F3_BQ - 1) / F3_BQ) * H * B;
    const int64_t blocks5 = ((S + F5_BQ - 1) / F5_BQ) * H * B;
    const int pin = kernel_override(LAVA_HIP_FAMILY_ATTN);
    const bool fast3 = lay_ok && scale > 0.f && (D == 64 || D == FA_D) && pin == 3 && blocks3 <= 0x7fffffff;
    const bool fast5 = lay_ok && !fast3 && blocks5 <= 0x7fffffff;
    // 128 < D <= 256 (a multiple of 8) with a positive scale: the ping-pong kernel over Q/K rows
    // zero-padded to 256, once per 128-column half of V and O (the scores are computed twice)
    bool fast256 = D > FA_D && D <= 256 && D % 8 == 0 && scale > 0.f && strides[0] == 1 && os[0] == 1 &&
                   blocks3 <= 0x7fffffff &&
                   aligned(Q, 16) && aligned(K, 16) && aligned(V, 16) && aligned(O, 8) &&
                   S * strides[1] * 2 < ((int64_t)1 << 31);
    for (int i = 1; i < 4; ++i) fast256 = fast256 && strides[i] % 8 == 0 && os[i] % 4 == 0;
    if (fast5) {   // any D <= 128, a multiple of 8 (staged zero-padded to 128; MFMAs over D rounded up to 64, 96, 128)
        auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, dim3((unsigned)blocks5), dim3(128 * F5_PAIRS), 0, s, p); };
        if (p.causal) {
            if (D <= 64) go(flash_fwd5_kernel<true, 64>);
            else if (D <= 96) go(flash_fwd5_kernel<true, 96>);
            else go(flash_fwd5_kernel<true, 128>);
        } else {
            if (D <= 64) go(flash_fwd5_kernel<false, 64>);
            else if (D <= 96) go(flash_fwd5_kernel<false, 96>);
            else go(flash_fwd5_kernel<false, 128>);
        }
        LAVA_LAUNCH_CHECK("flash_fwd5_kernel");
        return LAVA_HIP_OK;
    }
    if (fast3) {
        const dim3 grid((unsigned)blocks3);
        if (D == 64) {
            if (p.causal)
                hipLaunchKernelGGL((flash_fwd3_kernel<true, 64, 64>), grid, dim3(64 * F3_WAVES), 0, s, p);
            else
                hipLaunchKernelGGL((flash_fwd3_kernel<false, 64, 64>), grid, dim3(64 * F3_WAVES), 0, s, p);
        } else if (p.causal) {
            hipLaunchKernelGGL((flash_fwd3_kernel<true, 128, 128>), grid, dim3(64 * F3_WAVES), 0, s, p);
        } else {
            hipLaunchKernelGGL((flash_fwd3_kernel<false, 128, 128>), grid, dim3(64 * F3_WAVES), 0, s, p);
        }
        LAVA_LAUNCH_CHECK("flash_fwd3_kernel");
        return LAVA_HIP_OK;
    }
    if (fast256) {
        // two launches, each over the full 256-wide scores and one 128-column half of V and O
        const dim3 grid((unsigned)blocks3);
        for (int half = 0; half < 2; ++half) {
            FaParams ph = p;
            ph.V = p.V + 128 * half;
            ph.O = p.O + 128 * half;
            ph.dv = (int)(D - 128 * half < 128 ? D - 128 * half : 128);
            if (p.causal)
                hipLaunchKernelGGL((flash_fwd3_kernel<true, 256, 128>), grid, dim3(64 * F3_WAVES), 0, s, ph);
            else
                hipLaunchKernelGGL((flash_fwd3_kernel<false, 256, 128>), grid, dim3(64 * F3_WAVES), 0, s, ph);
            LAVA_LAUNCH_CHECK("flash_fwd3_kernel");
        }
        return LAVA_HIP_OK;
    }
    const int64_t rows = S * H * B;
    LAVA_REQUIRE((rows + 63) / 64 <= 0x7fffffff, LAVA_HIP_ERR_UNSUPPORTED, "flash_attn_fwd_f16: problem too large");
    hipLaunchKernelGGL(flash_generic_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, p, (int)D);
    LAVA_LAUNCH_CHECK("flash_generic_kernel");
    return LAVA_HIP_OK;
}
