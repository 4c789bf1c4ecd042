// Plain GEMMs on hipBLASLt: C[m, n] (+)= act(A[m, :k] . W[n, :k]^T + bias[n]) with row-major A, W and
// C, the contract of Kernels.gemm (J/tornado/Kernels.java:50-103) and the reference's cuBLAS path
// (Chronos2Forward.java:377-409). Row-major C = A W^T is the column-major product C^T = W A^T, so W
// is hipBLASLt's transposed first operand and A its second.
//
// The epilogue order is the reference's: bias, then the activation, then the accumulation. hipBLASLt
// applies its epilogue after alpha * W A^T + beta * C, so an activation with ACCUMULATE is declined
// (the caller runs its own kernel); BIAS with ACCUMULATE only reorders two additions. C in fp16 is
// declined too: the reference's FP16 twins saturate to +-65504 (Kernels.java:42-46), hipBLASLt's
// conversion does not.
//
// Results are reproducible: a plan replays the same task graph as the eager forward
// (J/chronos2/tornado/Chronos2Forward.java:292-300), so the same GEMM on the same operands must give
// the same bits whenever and on whichever stream it runs. On gfx950 hipBLASLt's kernels are Stream-K
// kernels ("..._SK3_..."): given a workspace, one may split a tile's k range over workgroups and
// combine the partial tiles through it. Only algorithms whose heuristic result needs no workspace are
// taken, and hipblasLtMatmul gets none (a null pointer and 0 bytes), so every tile of C is computed by
// one workgroup in a fixed order over k. A test checks that consequence: permuting the rows of A
// permutes the rows of C bit for bit, which a split k range would not keep.
//
// Per context: one handle and a cache of descriptors and the chosen algorithm per GEMM shape, so a
// call costs one descriptor update and the launch.
#include "jc_blas.hpp"

#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/jitcast_hip.h"

namespace jc {

namespace {

struct Key {
    int m, n, k, lda, ldc, ab, cd, epi, acc;
    bool operator==(const Key& o) const { return std::memcmp(this, &o, sizeof(Key)) == 0; }
};
struct KeyHash {
    size_t operator()(const Key& k) const {
        size_t h = 1469598103934665603ull;
        const unsigned char* p = reinterpret_cast<const unsigned char*>(&k);
        for (size_t i = 0; i < sizeof(Key); i++) h = (h ^ p[i]) * 1099511628211ull;
        return h;
    }
};

struct Entry {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;  // the heuristic offered a reproducible algorithm
};

hipDataType hip_type(int dtype) {
    return dtype == JC_BF16 ? HIP_R_16BF : dtype == JC_F16 ? HIP_R_16F : HIP_R_32F;
}

}  // namespace

// Preferred kernels for the GEMMs of config 4's calls: the layer's six GEMMs at the forecast's 260- and
// 180-row calls and at the whole 5,120-row request in one call (m = 34,580, 23,940 and 680,960
// rows x 133 tokens), in fp32, bf16 and the f16x3 split; and for the Timestral block's bf16 GEMMs at
// config 3's shape (64 series x 1,024 tokens, m = 65,536, and x 1,025 after the block's bucketing,
// m = 65,600: q|k|v, gate and up writing bf16, o and down accumulating fp32; and where they gained
// 3% or more, its fp32 and f16x3 GEMMs at the same counts; and the same for the Timestral
// forecast engine's blocks of 64 series x 1,028 tokens, m = 65,792), chosen by timing
// every workspace-free candidate of the hipBLASLt that the Python host maps (torch's bundled copy)
// on an MI355X; each comment gives the share of the time the kernel saved against the heuristic's
// first workspace-free candidate. A preference applies only to its exact shape and only where the named
// kernel is among that shape's workspace-free candidates, so the choice remains a function of the
// shape and the library (another hipBLASLt build keeps the first workspace-free candidate).
struct Pref {
    int m, n, k, ab, cd, epi, acc;
    const char* name;
};
static const Pref kPrefs[] = {
    {34580, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // f32 qkv: 4.3%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x144x32_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT4_9_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {34580, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 o: 4.1%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x144x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB1_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT4_9_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {34580, 3072, 768, 0, 0, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // f32 up: 14.1%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT128x224x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {34580, 768, 3072, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 down: 6.8%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT96x224x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT3_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {34580, 2304, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // bf16 qkv: 16.4%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {34580, 768, 768, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // bf16 o: 6.3%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT256x144x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT4_9_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {34580, 3072, 2304, 2, 0, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // x3 up: 5.6%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // f32 qkv: 10.7%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x96x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_3_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 o: 9.4%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT128x192x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB256_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT4_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 3072, 768, 0, 0, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // f32 up: 10.9%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x96x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_3_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 768, 3072, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 down: 5.7%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x96x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT8_3_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 2304, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // bf16 qkv: 12.4%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {23940, 768, 768, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // bf16 o: 23.2%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 3072, 768, 1, 1, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // bf16 up: 8.4%
     "Cijk_Alik_Bljk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT256x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA1024_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT8_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW8_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA8_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 768, 3072, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // bf16 down: 17.5%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 2304, 2304, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // x3 qkv: 5.5%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 768, 2304, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // x3 o: 19.1%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {23940, 768, 9216, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // x3 down: 13.3%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x192x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_6_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB2_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // f32 qkv: 10.5%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT96x224x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT3_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 o: 9.5%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT96x224x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT3_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 3072, 768, 0, 0, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // f32 up: 15.7%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT128x224x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 768, 3072, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // f32 down: 3.0%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT96x224x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT3_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 2304, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // bf16 qkv: 4.7%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {680960, 3072, 768, 1, 1, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // bf16 up: 12.9%
     "Cijk_Alik_Bljk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT192x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 3072, 2304, 2, 0, HIPBLASLT_EPILOGUE_RELU_BIAS, 0,  // x3 up: 14.0%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {680960, 768, 9216, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // x3 down: 3.5%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT96x160x128_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT3_5_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65536, 768, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral bf16 gate: 3.0%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65536, 6144, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral bf16 up: 11.0%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65600, 2304, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral bf16 qkv: 33.0%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65600, 768, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral bf16 gate: 5.4%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65600, 768, 768, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral bf16 o: 6.3%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT256x208x64_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT4_13_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {65600, 6144, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral bf16 up: 31.2%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65536, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral f32 qkv: 4.3%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x256x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_8_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB4_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65536, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral f32 gate: 7.3%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x128x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_4_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB4_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65536, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral f32 o: 5.5%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x128x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB512_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT8_4_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB4_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65536, 6144, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral f32 up: 4.1%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x256x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB256_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_8_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB4_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65536, 6144, 2304, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral x3 up: 5.3%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x256x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB1024_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_8_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB8_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65600, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral f32 qkv: 3.0%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x160x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_5_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65600, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral f32 gate: 9.4%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x160x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_5_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65600, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral f32 o: 7.8%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x160x32_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB4_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT8_5_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 2304, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast bf16 qkv: 35.7%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65792, 768, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast bf16 gate: 19.2%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65792, 768, 768, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral forecast bf16 o: 5.9%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT128x224x64_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 6144, 768, 1, 1, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast bf16 up: 20.8%
     "Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs_shortname0_gfx950"},
    {65792, 768, 3072, 1, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral forecast bf16 down: 5.5%
     "Cijk_Alik_Bljk_BSS_BH_Bias_S_HA_S_SAV_UserArgs_MT160x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT5_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 2304, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast f32 qkv: 6.3%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT128x224x16_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast f32 gate: 10.4%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x112x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {65792, 768, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral forecast f32 o: 8.9%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x112x32_MI16x16x1_SN_LDSB1_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA4_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA512_LBSPPB128_LBSPPM0_LPA8_LPB8_LPM0_LRVW4_LWPMn1_MIAV0_MIWT4_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG64_4_1"},
    {65792, 6144, 768, 0, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast f32 up: 27.6%
     "Cijk_Alik_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT256x224x16_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA2_GRVWB2_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA2_LPB2_LPM0_LRVW2_LWPMn1_MIAV0_MIWT8_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW4_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA4_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 2304, 2304, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 0,  // Timestral forecast x3 qkv: 16.1%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT192x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA256_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT6_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW2_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA2_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 768, 2304, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral forecast x3 o: 3.1%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT160x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT5_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
    {65792, 768, 9216, 2, 0, HIPBLASLT_EPILOGUE_DEFAULT, 1,  // Timestral forecast x3 down: 11.8%
     "Cijk_Alik_Bljk_HSS_BH_Bias_S_HA_S_SAV_UserArgs_MT160x224x64_MI16x16x1_SN_LDSB0_AFC1_AFEM1_AFEM1_ASEM1_CLR1_CADS0_DTVA0_DTVB0_EPS0_FDSI0_GRPM1_GRVWA8_GRVWB8_GSU0_GSUAMB_GLS0_ISA950_IU1_K1_LBSPPA128_LBSPPB128_LBSPPM0_LPA16_LPB16_LPM0_LRVW8_LWPMn1_MIAV0_MIWT5_7_MO40_NTn1_NTA0_NTB0_NTC0_NTD0_NTM0_NEPBS0_NLCA1_NLCB1_ONLL1_PGR2_PLR1_PKA1_SIA3_SS1_SPO0_SRVW0_SSO0_SVW1_SK3_SKXCCM8_TLDS1_ULSGRO0_USL1_UIOFGRO0_USFGRO0_VSn1_VWA1_VWB1_WSGRA0_WSGRB0_WS64_WG32_8_1"},
};

static const char* preferred(const Key& key) {
    for (const Pref& p : kPrefs)
        if (p.m == key.m && p.n == key.n && p.k == key.k && p.ab == key.ab && p.cd == key.cd && p.epi == key.epi &&
            p.acc == key.acc)
            return p.name;
    return nullptr;
}

// an activation without a bias runs as activation-with-bias on zeros (x + 0 = x exactly): hipBLASLt
// has more algorithms for the bias forms
constexpr int kZeroBias = 1 << 16;

struct Blas {
    hipblasLtHandle_t handle = nullptr;
    float* zeros = nullptr;  // kZeroBias floats
    std::unordered_map<Key, Entry, KeyHash> cache;
    std::unordered_set<uint64_t> reported;  // declined shapes already reported (JITCAST_HIP_BLAS_DEBUG)
};

Blas* blas_create() {
    Blas* b = new (std::nothrow) Blas();
    if (!b) return nullptr;
    if (hipblasLtCreate(&b->handle) != HIPBLAS_STATUS_SUCCESS) {
        delete b;
        return nullptr;
    }
    if (hipMalloc(&b->zeros, kZeroBias * sizeof(float)) != hipSuccess ||
        hipMemset(b->zeros, 0, kZeroBias * sizeof(float)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(b->zeros);
        (void)hipblasLtDestroy(b->handle);
        delete b;
        return nullptr;
    }
    return b;
}

void blas_destroy(Blas* b) {
    if (!b) return;
    for (auto& kv : b->cache) {
        Entry& e = kv.second;
        if (e.desc) (void)hipblasLtMatmulDescDestroy(e.desc);
        if (e.lw) (void)hipblasLtMatrixLayoutDestroy(e.lw);
        if (e.la) (void)hipblasLtMatrixLayoutDestroy(e.la);
        if (e.lc) (void)hipblasLtMatrixLayoutDestroy(e.lc);
    }
    (void)hipFree(b->zeros);
    (void)hipblasLtDestroy(b->handle);
    delete b;
}

// JITCAST_HIP_BLAS_DEBUG=1 reports on stderr the kernel chosen for each GEMM shape and each shape this
// path declines, once per shape and context.
static bool debug_on() {
    static const bool on = [] {
        const char* e = getenv("JITCAST_HIP_BLAS_DEBUG");
        return e && *e == '1';
    }();
    return on;
}

static Entry* entry_for(Blas* b, const Key& key) {
    auto it = b->cache.find(key);
    if (it != b->cache.end()) return &it->second;
    Entry e;
    const hipDataType ab = hip_type(key.ab), cd = hip_type(key.cd);
    bool good = hipblasLtMatmulDescCreate(&e.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    if (good) {
        const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
        const hipblasLtEpilogue_t epi = (hipblasLtEpilogue_t)key.epi;
        good = hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == 0 &&
               hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == 0 &&
               hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof epi) == 0;
        if (good && (key.epi & HIPBLASLT_EPILOGUE_BIAS)) {
            // the support check below wants a bias pointer; each call sets its own before the launch
            const hipDataType bt = HIP_R_32F;
            const float* placeholder = b->zeros;
            good = hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt) == 0 &&
                   hipblasLtMatmulDescSetAttribute(e.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &placeholder,
                                                   sizeof placeholder) == 0;
        }
    }
    // W: column-major k x n (ld k); A: column-major k x m (ld lda); C: column-major n x m (ld ldc)
    good = good && hipblasLtMatrixLayoutCreate(&e.lw, ab, key.k, key.n, key.k) == 0 &&
           hipblasLtMatrixLayoutCreate(&e.la, ab, key.k, key.m, key.lda) == 0 &&
           hipblasLtMatrixLayoutCreate(&e.lc, cd, key.n, key.m, key.ldc) == 0;
    if (good) {
        hipblasLtMatmulPreference_t pref = nullptr;
        if (hipblasLtMatmulPreferenceCreate(&pref) == 0) {
            // the heuristic ranks its candidates as if any workspace were available; each one's need for
            // this very problem then comes from matmulIsAlgoSupported, and the shape's preferred kernel
            // (kPrefs) or else the first that needs none is taken. The choice is a function of the
            // shape alone: every context and process makes it.
            const uint64_t rank_as_if = 1ull << 30;
            // deep enough that a workspace-free candidate turns up: for config 4's fp32 shapes the
            // first one ranks 9th to 50th, within 0-11% of the heuristic's first choice
            constexpr int kAsk = 512;
            std::vector<hipblasLtMatmulHeuristicResult_t> res;
            try {
                res.resize(kAsk);
            } catch (...) {
                res.clear();
            }
            int got = 0;
            const float alpha = 1.f, beta = key.acc ? 1.f : 0.f;
            if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &rank_as_if,
                                                      sizeof rank_as_if) == 0 &&
                !res.empty() &&
                hipblasLtMatmulAlgoGetHeuristic(b->handle, e.desc, e.lw, e.la, e.lc, e.lc, pref, kAsk, res.data(), &got) == 0) {
                auto free_of_workspace = [&](int i) {
                    size_t need = 1;
                    const hipblasStatus_t sup =
                        res[i].state != HIPBLAS_STATUS_SUCCESS
                            ? res[i].state
                            : hipblaslt_ext::matmulIsAlgoSupported(b->handle, e.desc, &alpha, e.lw, e.la, &beta, e.lc,
                                                                   e.lc, res[i].algo, need);
                    return sup == HIPBLAS_STATUS_SUCCESS && need == 0;
                };
                auto kernel_name = [&](hipblasLtMatmulAlgo_t algo) {
                    try {
                        return hipblaslt_ext::getKernelNameFromAlgo(b->handle, algo);
                    } catch (...) {
                        return std::string("?");
                    }
                };
                // the shape's preferred kernel, where it is a workspace-free candidate
                if (const char* want = preferred(key)) {
                    for (int i = 0; i < got && !e.ok; i++) {
                        if (kernel_name(res[i].algo) != want || !free_of_workspace(i)) continue;
                        e.algo = res[i].algo;
                        e.ok = true;
                        if (debug_on())
                            fprintf(stderr, "[jc_blas] m=%d n=%d k=%d ab=%d c=%d epi=%d acc=%d: %s (preferred, candidate "
                                    "%d of %d)\n", key.m, key.n, key.k, key.ab, key.cd, key.epi, key.acc, want, i + 1, got);
                    }
                }
                int skipped = 0;
                for (int i = 0; i < got && !e.ok; i++) {
                    if (!free_of_workspace(i)) {
                        skipped++;
                        continue;
                    }
                    e.algo = res[i].algo;
                    e.ok = true;
                    if (debug_on()) {
                        const std::string name = kernel_name(e.algo);
                        fprintf(stderr, "[jc_blas] m=%d n=%d k=%d ab=%d c=%d epi=%d acc=%d: %s (candidate %d of %d; %d "
                                "skipped: unsupported or needing a workspace)\n", key.m, key.n, key.k, key.ab, key.cd,
                                key.epi, key.acc, name.c_str(), i + 1, got, skipped);
                    }
                }
            }
            (void)hipblasLtMatmulPreferenceDestroy(pref);
        }
    }
    try {
        return &b->cache.emplace(key, e).first->second;
    } catch (...) {
        return nullptr;
    }
}

static BlasStatus decline(Blas* b, const char* why, int m, int n, int k, int flags, int ab, int cd) {
    if (debug_on()) {
        uint64_t h = 1469598103934665603ull;
        for (int v : {m, n, k, flags, ab, cd}) h = (h ^ (uint32_t)v) * 1099511628211ull;
        bool fresh = true;
        try {
            fresh = b->reported.insert(h).second;
        } catch (...) {
        }
        if (fresh)
            fprintf(stderr, "[jc_blas] declined m=%d n=%d k=%d flags=%d ab=%d c=%d: %s\n", m, n, k, flags, ab, cd, why);
    }
    return kBlasDecline;
}

BlasStatus blas_gemm(Blas* b, const void* a, int lda, const void* w, const float* bias, void* c, int ldc, int m, int n,
                     int k, int flags, int ab_dtype, int c_dtype, hipStream_t stream) {
    if (!b) return kBlasDecline;
    const bool act = flags & (JC_GEMM_RELU | JC_GEMM_SILU);
    const bool acc = flags & JC_GEMM_ACCUMULATE;
    if ((act && acc) || c_dtype == JC_F16) return decline(b, "combination", m, n, k, flags, ab_dtype, c_dtype);
    if (c_dtype != JC_F32 && c_dtype != ab_dtype) return decline(b, "output type", m, n, k, flags, ab_dtype, c_dtype);
    bool has_bias = (flags & JC_GEMM_BIAS) && bias;
    if (act && !has_bias) {
        if (n > kZeroBias) return decline(b, "activation without a bias", m, n, k, flags, ab_dtype, c_dtype);
        bias = b->zeros;
        has_bias = true;
    }
    int epi = HIPBLASLT_EPILOGUE_DEFAULT;
    if (flags & JC_GEMM_RELU) epi = has_bias ? HIPBLASLT_EPILOGUE_RELU_BIAS : HIPBLASLT_EPILOGUE_RELU;
    else if (flags & JC_GEMM_SILU) epi = has_bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT;
    else if (has_bias) epi = HIPBLASLT_EPILOGUE_BIAS;
    const Key key{m, n, k, lda, ldc, ab_dtype, c_dtype, epi, acc ? 1 : 0};
    Entry* e = entry_for(b, key);
    if (!e || !e->ok) return decline(b, "no algorithm", m, n, k, flags, ab_dtype, c_dtype);
    if (has_bias &&
        hipblasLtMatmulDescSetAttribute(e->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias) != 0)
        return kBlasError;
    const float alpha = 1.f, beta = acc ? 1.f : 0.f;
    const hipblasStatus_t s = hipblasLtMatmul(b->handle, e->desc, &alpha, w, e->lw, a, e->la, &beta, c, e->lc, c,
                                              e->lc, &e->algo, nullptr, 0, stream);
    return s == HIPBLAS_STATUS_SUCCESS ? kBlasDone : kBlasError;
}

}  // namespace jc
