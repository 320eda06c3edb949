// flash_attn.hip -- causal flash-attention forward, fp16 in/out, fp32 softmax state.
//
// The reference is the coopmat2 flash kernel Lava's vocabulary was shaped for
// (`attn_flash_rows!` / flash_attn_cm2, src/vocabulary/coopmat.jl:158;
// src/device/coopmat_intrinsics.jl:535-755): per query block, per key block,
//   S = Q K^T; rowmax = reduce(max, S, Row); M = max(rowmax, Mold);
//   P = exp(S - M); O = O * exp(Mold - M) + P V; L = L * exp(Mold - M) + rowsum(P)
// and finally O / L, converted to fp16 (RNE).
//
// CDNA4 formulation (one wavefront = 32 queries, 4 wavefronts = 128 queries):
//  * everything is computed transposed, S^T = K Q^T and O^T = V^T P^T, with the
//    32x32x16 fp16 MFMA.  In that form the accumulator lane owns ONE query
//    (lane % 32; lanes l and l ^ 32 share it) and holds that query's scores for
//    16 keys per 32-key tile, so the row max and row sum are in-lane reductions
//    plus one exchange with lane ^ 32, the rescale of O is one multiplier per
//    lane, and the score accumulator is directly the B operand P^T of the second
//    product (keys in-lane), with no relayout through LDS;
//  * Q^T stays in registers for the whole key loop (8 x 16 bytes per lane);
//  * K and V tiles of 64 keys are double-buffered in LDS; K as [key][d] with the
//    16-byte chunks XOR-swizzled by key % 16 (the fragment read of 32 keys x one
//    chunk then hits every bank once), V transposed to [d][key] (row pitch 136 B)
//    so that the A operand V^T reads 4 consecutive keys per 8-byte access;
//  * softmax in base 2: s * (scale * log2 e), v_exp_f32;
//  * causal: key blocks above the diagonal are never loaded, the two diagonal
//    blocks are masked per element, and a wavefront skips the products of a block
//    that lies entirely above its 32 queries;
//  * workgroups are ordered XCD by XCD so that all query blocks of one (batch,
//    head) run on one XCD and share its K and V through that XCD's L2, longest
//    query blocks first.
#include <hip/hip_runtime.h>

#include "lava_coopmat.hpp"
#include "lava_hip_internal.hpp"

namespace lava {

constexpr int FA_D = 128;
constexpr int FA_BQ = 128;
constexpr int FA_BK = 64;
constexpr int FA_K_BYTES = FA_BK * FA_D * 2;     // 16 KB
constexpr int FA_VT_PITCH = FA_BK * 2 + 8;       // 136 B per d-row of V^T
constexpr int FA_VT_BYTES = FA_D * FA_VT_PITCH;  // 17 KB

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
};

__device__ __forceinline__ float wave_xor32_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }

template <bool CAUSAL>
__global__ void __launch_bounds__(256, 2) flash_fwd_kernel(FaParams p) {
    __shared__ __attribute__((aligned(16))) uint8_t k_lds[2][FA_K_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t vt_lds[2][FA_VT_BYTES];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nqb = p.S / FA_BQ;
    const int nbh = p.H * p.B;
    // workgroup -> (batch*head, query block): consecutive ids on one XCD, heavy first
    int bid = blockIdx.x, bh, qb;
    const int total = nqb * nbh;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    bh = bid / nqb;
    qb = CAUSAL ? (nqb - 1 - bid % nqb) : bid % nqb;
    const int h = bh % p.H, b = bh / p.H;

    const f16* Qb = p.Q + h * p.sh + b * p.sb;
    const f16* Kb = p.K + h * p.sh + b * p.sb;
    const f16* Vb = p.V + h * p.sh + b * p.sb;
    f16* Ob = p.O + h * p.osh + b * p.osb;

    const int q0 = qb * FA_BQ + w * 32;       // this wave's first query
    const int qi = lane & 31, h2 = lane >> 5;
    const int my_q = q0 + qi;

    // Q^T as B operand: lane (query qi, half h2) holds d = 16 ks + 8 h2 + [0, 8)
    uint4 qf[8];
    {
        const f16* qrow = Qb + (int64_t)my_q * p.sl + 8 * h2;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) qf[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
    }

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
    float m_run = -3.0e38f;   // the reference's initial running maximum
    float l_run = 0.f;        // this lane's partial row sum (keys held by this lane)

    const int nkb = CAUSAL ? (qb * FA_BQ + FA_BQ) / FA_BK : p.S / FA_BK;

    // ---- global -> registers -> LDS staging of one key block
    // K: 64 keys x 16 chunks of 16 B; thread handles chunks tid + 256 i.
    // V: key pairs (2 pp, 2 pp + 1) x chunk c; thread handles items tid + 256 i.
    uint4 kreg[4], vreg[2][2];
    auto load_block = [&](int kb) {
        const int key0 = kb * FA_BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int item = tid + 256 * i, key = item >> 4, c = item & 15;
            kreg[i] = *reinterpret_cast<const uint4*>(Kb + (int64_t)(key0 + key) * p.sl + 8 * c);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int item = tid + 256 * i, pp = item & 31, c = item >> 5;
            const f16* vp = Vb + (int64_t)(key0 + 2 * pp) * p.sl + 8 * c;
            vreg[i][0] = *reinterpret_cast<const uint4*>(vp);
            vreg[i][1] = *reinterpret_cast<const uint4*>(vp + p.sl);
        }
    };
    auto store_block = [&](int stage) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int item = tid + 256 * i, key = item >> 4, c = item & 15;
            *reinterpret_cast<uint4*>(&k_lds[stage][key * 256 + ((c ^ (key & 15)) << 4)]) = kreg[i];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int item = tid + 256 * i, pp = item & 31, c = item >> 5;
            const uint32_t* a = reinterpret_cast<const uint32_t*>(&vreg[i][0]);
            const uint32_t* bq = reinterpret_cast<const uint32_t*>(&vreg[i][1]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // (V[2pp][8c + e], V[2pp + 1][8c + e]) -> V^T[8c + e][2pp .. 2pp + 1]
                const uint32_t lo = (a[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                const uint32_t hi = (bq[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                *reinterpret_cast<uint32_t*>(&vt_lds[stage][(8 * c + e) * FA_VT_PITCH + 4 * pp]) = lo | (hi << 16);
            }
        }
    };

    load_block(0);
    store_block(0);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const int stage = kb & 1;
        const bool has_next = kb + 1 < nkb;
        if (has_next) load_block(kb + 1);
        const int key0 = kb * FA_BK;
        // a wave whose 32 queries all precede this block has nothing to add
        const bool active = !CAUSAL || key0 <= q0 + 31;
        if (active) {
            // ---- S^T = K Q^T: 2 key tiles of 32
            f32x16 st[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int r = 0; r < 16; ++r) st[kt][r] = 0.f;
                const int key = kt * 32 + qi;   // A operand row
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    const int c = 2 * ks + h2;
                    const uint4 kf = *reinterpret_cast<const uint4*>(&k_lds[stage][key * 256 + ((c ^ (key & 15)) << 4)]);
                    st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, kf),
                                                                    __builtin_bit_cast(f16x8, qf[ks]), st[kt], 0, 0, 0);
                }
            }
            // ---- scale, mask, running max.  st[kt][r] is key key0 + 32 kt + 8 (r / 4) + 4 h2 + r % 4.
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float s = st[kt][r] * p.scale_log2;
                    if (CAUSAL) {
                        const int key = key0 + 32 * kt + 8 * (r >> 2) + 4 * h2 + (r & 3);
                        if (key > my_q) s = -INFINITY;
                    }
                    st[kt][r] = s;
                    mx = fmaxf(mx, s);
                }
            mx = wave_xor32_max(mx);
            const float m_new = fmaxf(m_run, mx);
            const float alpha = exp2f(m_run - m_new);
            m_run = m_new;
            float lsum = 0.f;
            uint4 pf[2][2];   // P^T as B operand: [kt][ks], 8 fp16 each
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    f16x8 pv;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float e = exp2f(st[kt][8 * ks + i] - m_new);
                        lsum += e;
                        pv[i] = (f16)e;
                    }
                    pf[kt][ks] = __builtin_bit_cast(uint4, pv);
                }
            l_run = l_run * alpha + lsum;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            // ---- O^T += V^T P^T.  B slot i of (kt, ks) is key 32 kt + 16 ks + 8 (i / 4) + 4 h2 + i % 4,
            // so the A operand lane (d, h2) reads keys [32 kt + 16 ks + 4 h2, +4) and [.. + 8, +4) of V^T row d.
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint8_t* vrow = &vt_lds[stage][(dt * 32 + qi) * FA_VT_PITCH];
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const int kk = 32 * kt + 16 * ks + 4 * h2;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 2 * kk);
                        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 2 * (kk + 8));
                        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
                        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, vf),
                                                                       __builtin_bit_cast(f16x8, pf[kt][ks]), o[dt], 0,
                                                                       0, 0);
                    }
            }
        }
        if (has_next) store_block(stage ^ 1);
        __syncthreads();
    }

    // ---- O / L, fp16, store.  o[dt][r] is d = 32 dt + 8 (r / 4) + 4 h2 + r % 4 of query my_q.
    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const float inv = 1.f / l_tot;
    f16* orow = Ob + (int64_t)my_q * p.osl;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int d = 32 * dt + 8 * g4 + 4 * h2;
            f16x4 v = {(f16)(o[dt][4 * g4 + 0] * inv), (f16)(o[dt][4 * g4 + 1] * inv), (f16)(o[dt][4 * g4 + 2] * inv),
                       (f16)(o[dt][4 * g4 + 3] * inv)};
            *reinterpret_cast<f16x4*>(orow + d) = v;
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
    hipStream_t s = as_stream(stream);

    bool fast = D == FA_D && S % FA_BQ == 0;
    for (int i = 1; i < 4; ++i) fast = fast && strides[i] % 8 == 0 && os[i] % 4 == 0;
    fast = fast && aligned(Q, 16) && aligned(K, 16) && aligned(V, 16) && aligned(O, 8);
    const int64_t blocks = (S / FA_BQ) * H * B;
    fast = fast && blocks <= 0x7fffffff;
    if (fast) {
        if (p.causal)
            hipLaunchKernelGGL(flash_fwd_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(flash_fwd_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        LAVA_LAUNCH_CHECK("flash_fwd_kernel");
        return LAVA_HIP_OK;
    }
    const int64_t rows = S * H * B;
    LAVA_REQUIRE((rows + 63) / 64 <= 0x7fffffff, LAVA_HIP_ERR_UNSUPPORTED, "flash_attn_fwd_f16: problem too large");
    hipLaunchKernelGGL(flash_generic_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, p, (int)D);
    LAVA_LAUNCH_CHECK("flash_generic_kernel");
    return LAVA_HIP_OK;
}
