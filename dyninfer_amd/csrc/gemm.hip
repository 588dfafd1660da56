// Prefill GEMM: launch planning and dispatch (host side).  The kernels are in
// gemm_impl.hpp, instantiated per encoding in gemm_<enc>.hip.
#include "gemm_impl.hpp"

#include <algorithm>

namespace dmx {
namespace gemm {

extern template hipError_t launch_plan<ENC_Q4_0>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_Q4_1>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_Q8_0>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_Q6_K>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_Q4_K>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_Q5_K>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_IQ4_XS>(const GemmArgs&, const GemmPlan&, hipStream_t);
extern template hipError_t launch_plan<ENC_MLX_U4>(const GemmArgs&, const GemmPlan&, hipStream_t);

namespace {

bool fits_enc(uint32_t enc, int tm, int nb, int s) {
    switch (enc) {
        case ENC_Q4_0: return fits<ENC_Q4_0>(tm, nb, s);
        case ENC_Q4_1: return fits<ENC_Q4_1>(tm, nb, s);
        case ENC_Q8_0: return fits<ENC_Q8_0>(tm, nb, s);
        case ENC_Q6_K: return fits<ENC_Q6_K>(tm, nb, s);
        case ENC_Q4_K: return fits<ENC_Q4_K>(tm, nb, s);
        case ENC_Q5_K: return fits<ENC_Q5_K>(tm, nb, s);
        case ENC_IQ4_XS: return fits<ENC_IQ4_XS>(tm, nb, s);
        case ENC_MLX_U4: return fits<ENC_MLX_U4>(tm, nb, s);
        default: return false;
    }
}

// Decode VALU instructions per (N-block, k step) per lane, from the kernels'
// ISA: the encoding's term in the cost model.
double dec_cost(uint32_t enc) {
    switch (enc) {
        case ENC_Q8_0: return 18.0;
        case ENC_Q6_K: return 30.0;
        case ENC_Q4_K: return 22.0;
        case ENC_Q5_K:
        case ENC_IQ4_XS: return 28.0;
        default: return 16.0;  // Q4_0, Q4_1, MLX U4
    }
}

}  // namespace
}  // namespace gemm

using gemm::GemmArgs;

uint32_t gemm_layout(uint32_t enc) {
    switch (enc) {
        case ENC_Q4_0:
        case ENC_Q4_1: return XFRAG_NIB;
        case ENC_Q8_0: return XFRAG_BYTE;
        case ENC_Q6_K: return XFRAG_BYTE;  // a lane's 32 codes in order, as Q8_0
        case ENC_Q4_K:
        case ENC_Q5_K: return XFRAG_BYTE;
        case ENC_IQ4_XS: return XFRAG_NIB;  // a sub-block laid out as a Q4_0 block
        case ENC_MLX_U4: return XFRAG_WORD;
        default: return ~0u;
    }
}

bool gemm_supported(uint32_t enc, uint32_t N, uint32_t K, uint32_t M) {
    return gemm_layout(enc) != ~0u && N > 0 && M > 0 && K >= 64u &&
           K % (enc == ENC_Q6_K || enc == ENC_Q4_K || enc == ENC_Q5_K || enc == ENC_IQ4_XS ? 256u : 64u) == 0;
}

// Launch plan from a cost model fitted to graph-replayed calls (staging +
// GEMM) of every plan on 17 shapes (M 128..2048, N 1024..12288, K 1024..12288;
// Q4_0, Q6_K, Q4_K, Q8_0, MLX U4), in us per call:
//   t = 3.87 + rounds · (nc · (0.0712·TM·NB + 0.2074·NB·dec/16 + 0.0737)
//                        + 0.0987·TM·NB·(S > 1 ? 4 : 1) + 4.99)
// with nc the 64-k chunks per wave (K/64/S), rounds = ceil(workgroups / 256)
// (one workgroup per CU), dec the encoding's decode VALU per (N-block, k
// step); the last term is the epilogue's LDS round trip of the partial tiles.
// It picks the measured best plan on 16 of the 17 shapes and one within 1.2%
// on the other (MLX M512 N3072 K1024).  Candidates: TM 2 or 4 activation row
// blocks (4 only above 64 rows), NB 2 or 3 weight row blocks per wave, S 1, 2
// or 4 K slices per workgroup (those whose LDS fits, S dividing the chunks).
GemmPlan gemm_plan(uint32_t enc, uint32_t N, uint32_t K, uint32_t M) {
    const double dec = gemm::dec_cost(enc) / 16.0;
    const uint32_t mb = (M + 31u) / 32u, nchk = K / 64u;
    GemmPlan best{2, 2, 1, 0, 0};
    double best_t = 1e300;
    for (uint32_t tm : {4u, 2u}) {
        if (tm == 4u && mb <= 2u) continue;
        for (uint32_t nb : {3u, 2u}) {
            for (uint32_t s : {4u, 2u, 1u}) {
                if (!gemm::fits_enc(enc, (int)tm, (int)nb, (int)s) || nchk % s != 0) continue;
                const uint32_t wn = 4u / s;
                const uint32_t mt = (mb + tm - 1u) / tm, nt = (N + 32u * nb * wn - 1u) / (32u * nb * wn);
                const double nc = (double)(nchk / s), rounds = (double)(((uint64_t)mt * nt + 255u) / 256u);
                const double t = 3.87 + rounds * (nc * (0.0712 * tm * nb + 0.2074 * nb * dec + 0.0737) +
                                                   0.0987 * tm * nb * (s > 1u ? 4.0 : 1.0) + 4.99);
                if (t < best_t * 0.999) {
                    best_t = t;
                    best = {tm, nb, s, mt, nt};
                }
            }
        }
    }
    return best;
}

hipError_t gemm_launch(const GemmWeight& wt, uint32_t N, uint32_t K, const uint16_t* xh, const float* rs, uint32_t M,
                       void* y, bool y_bf16, hipStream_t st) {
    const uint32_t enc = wt.enc;
    if (!gemm_supported(enc, N, K, M)) return hipErrorInvalidValue;
    if (enc == ENC_MLX_U4 && (wt.group == 0 || wt.group % 32u || K % wt.group || wt.sdtype > DT_BF16 || !wt.sc || !wt.bi))
        return hipErrorInvalidValue;
    const GemmPlan p = gemm_plan(enc, N, K, M);
    GemmArgs a{};
    a.w = wt.w;
    a.xh = xh;
    a.rs = rs;
    a.y = y;
    a.M = M;
    a.N = N;
    a.K = K;
    a.mt = p.mt;
    a.nt = p.nt;
    a.y_bf16 = y_bf16 ? 1u : 0u;
    a.sc = wt.sc;
    a.bi = wt.bi;
    a.group = wt.group;
    a.gmagic = group_magic(wt.group);
    a.sdtype = wt.sdtype;
    switch (enc) {
        case ENC_Q4_0: a.rowbytes = (uint64_t)(K / 32u) * 18u; break;
        case ENC_Q4_1: a.rowbytes = (uint64_t)(K / 32u) * 20u; break;
        case ENC_Q8_0: a.rowbytes = (uint64_t)(K / 32u) * 34u; break;
        case ENC_Q6_K: a.rowbytes = (uint64_t)(K / 256u) * 210u; break;
        case ENC_Q4_K: a.rowbytes = (uint64_t)(K / 256u) * 144u; break;
        case ENC_Q5_K: a.rowbytes = (uint64_t)(K / 256u) * 176u; break;
        case ENC_IQ4_XS: a.rowbytes = (uint64_t)(K / 256u) * 136u; break;
        default: a.rowbytes = (uint64_t)K / 2u; break;  // MLX packed words (scales and biases besides)
    }
    // M-major tile order when the staged activations (2 bytes per element)
    // outweigh the weights (M2048 N3072 K1024: 34.3 against 35.9 us per call)
    a.mmajor = (uint64_t)M * K * 2u > (uint64_t)N * a.rowbytes ? 1u : 0u;
    switch (enc) {
        case ENC_Q4_0: return gemm::launch_plan<ENC_Q4_0>(a, p, st);
        case ENC_Q4_1: return gemm::launch_plan<ENC_Q4_1>(a, p, st);
        case ENC_Q8_0: return gemm::launch_plan<ENC_Q8_0>(a, p, st);
        case ENC_Q6_K: return gemm::launch_plan<ENC_Q6_K>(a, p, st);
        case ENC_Q4_K: return gemm::launch_plan<ENC_Q4_K>(a, p, st);
        case ENC_Q5_K: return gemm::launch_plan<ENC_Q5_K>(a, p, st);
        case ENC_IQ4_XS: return gemm::launch_plan<ENC_IQ4_XS>(a, p, st);
        case ENC_MLX_U4: return gemm::launch_plan<ENC_MLX_U4>(a, p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dmx
