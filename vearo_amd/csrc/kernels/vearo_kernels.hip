// vearo_kernels.hip -- the single translation unit compiled to the gfx950 code
// object (hipcc --genco) that libvearo_hip.so embeds and loads with
// hipModuleLoadData. Every kernel is extern "C" with one argument struct; the
// host looks kernels up by these names (see vearo_amd/csrc/runtime.cpp).
//
// Row-engine kernels are instantiated per (TEAM, NV, VW):
//   TEAM lanes own one row, each lane holds NV units of VW floats.
#include "common.h"
#include "embedding.h"
#include "gelu.h"
#include "gemm.h"
#include "gemm_big.h"
#include "generic.h"
#include "layernorm.h"
#include "optim.h"
#include "rowwide.h"
#include "softmax.h"
#include "xent.h"

#define BS_OF(T) ((T) > 256 ? (T) : 256)

// (TEAM, NV) pairs; NV <= 8 are also used by the backward kernels.
#define ROW_CFG_SMALL(M, VW) \
  M(16, 1, VW) M(32, 1, VW) M(64, 1, VW) M(64, 2, VW) M(64, 3, VW) M(64, 4, VW) \
  M(64, 6, VW) M(64, 8, VW) M(1024, 1, VW) M(1024, 2, VW) M(1024, 3, VW) \
  M(1024, 4, VW) M(1024, 6, VW) M(1024, 8, VW)
#define ROW_CFG_BIG(M, VW) M(64, 12, VW) M(64, 16, VW) M(1024, 12, VW) M(1024, 16, VW)
#define ROW_CFG_ALL(M, VW) ROW_CFG_SMALL(M, VW) ROW_CFG_BIG(M, VW)
// Sub-wave / wave teams with short rows also come in 2- and 4-rows-per-team forms.
#define ROW_CFG_MULTI(M, VW) \
  M(16, 1, VW) M(32, 1, VW) M(64, 1, VW) M(64, 2, VW) M(64, 3, VW) M(64, 4, VW)

#define K_LN_FWD_R(T, N, VW, R)                                                   \
  extern "C" __global__ void __launch_bounds__(BS_OF(T))                          \
      vh_ln_fwd_t##T##_n##N##_v##VW##_r##R(LnFwdArgs a) {                         \
    ln_fwd_impl<T, N, VW, R>(a);                                                  \
  }
#define K_LN_FWD(T, N, VW) K_LN_FWD_R(T, N, VW, 1)
#define K_LN_FWD_M(T, N, VW) K_LN_FWD_R(T, N, VW, 2) K_LN_FWD_R(T, N, VW, 4)
ROW_CFG_ALL(K_LN_FWD, 1)
ROW_CFG_ALL(K_LN_FWD, 4)
ROW_CFG_MULTI(K_LN_FWD_M, 1)
ROW_CFG_MULTI(K_LN_FWD_M, 4)
// Full-row forms (C == T * N * 4) of the wave-team configurations.
#define K_LN_FWD_F(T, N)                                                          \
  extern "C" __global__ void __launch_bounds__(BS_OF(T))                          \
      vh_ln_fwd_t##T##_n##N##_v4_r4_f(LnFwdArgs a) {                              \
    ln_fwd_impl<T, N, 4, 4, true>(a);                                             \
  }
K_LN_FWD_F(64, 1) K_LN_FWD_F(64, 2) K_LN_FWD_F(64, 3) K_LN_FWD_F(64, 4)

#define K_LN_BWD_B(T, N, VW, BS)                                                  \
  extern "C" __global__ void __launch_bounds__(BS)                                \
      vh_ln_bwd_t##T##_n##N##_v##VW##_b##BS(LnBwdArgs a) {                        \
    extern __shared__ float dyn_lds[];                                            \
    ln_bwd_impl<T, N, VW, BS>(a, dyn_lds);                                        \
  }
#define BSLIT_16 256
#define BSLIT_32 256
#define BSLIT_64 256
#define BSLIT_1024 1024
#define K_LN_BWD_X(T, N, VW, BS) K_LN_BWD_B(T, N, VW, BS)  // expands BS before pasting
#define K_LN_BWD(T, N, VW) K_LN_BWD_X(T, N, VW, BSLIT_##T)
#define K_LN_BWD_512(T, N, VW) K_LN_BWD_B(T, N, VW, 512)
ROW_CFG_SMALL(K_LN_BWD, 1)
// 128-bit units: rows held by 1024-thread teams up to 16 floats per lane (the
// 24- and 32-float forms spilled; longer rows take kernels/rowwide.h).
K_LN_BWD(16, 1, 4) K_LN_BWD(32, 1, 4) K_LN_BWD(64, 1, 4) K_LN_BWD(64, 2, 4) K_LN_BWD(64, 3, 4)
K_LN_BWD(64, 4, 4) K_LN_BWD(64, 6, 4) K_LN_BWD(64, 8, 4) K_LN_BWD(1024, 1, 4) K_LN_BWD(1024, 2, 4)
K_LN_BWD(1024, 3, 4) K_LN_BWD(1024, 4, 4)
// Wave teams with rows up to 1024 units: 8 row-groups per workgroup.
K_LN_BWD_512(64, 1, 1) K_LN_BWD_512(64, 2, 1) K_LN_BWD_512(64, 3, 1) K_LN_BWD_512(64, 4, 1)
K_LN_BWD_512(64, 1, 4) K_LN_BWD_512(64, 2, 4) K_LN_BWD_512(64, 3, 4) K_LN_BWD_512(64, 4, 4)
#define K_LN_BWD_F(T, N)                                                          \
  extern "C" __global__ void __launch_bounds__(512) vh_ln_bwd_t##T##_n##N##_v4_b512_f(LnBwdArgs a) { \
    extern __shared__ float dyn_lds[];                                            \
    ln_bwd_impl<T, N, 4, 512, true>(a, dyn_lds);                                  \
  }
K_LN_BWD_F(64, 1) K_LN_BWD_F(64, 2) K_LN_BWD_F(64, 3) K_LN_BWD_F(64, 4)

#define K_SM_FWD_R(T, N, VW, R)                                                   \
  extern "C" __global__ void __launch_bounds__(BS_OF(T))                          \
      vh_sm_fwd_t##T##_n##N##_v##VW##_r##R(SoftmaxArgs a) {                       \
    softmax_fwd_impl<T, N, VW, R>(a);                                             \
  }
#define K_SM_FWD(T, N, VW) K_SM_FWD_R(T, N, VW, 1)
#define K_SM_FWD_M(T, N, VW) K_SM_FWD_R(T, N, VW, 2)
ROW_CFG_ALL(K_SM_FWD, 1)
ROW_CFG_ALL(K_SM_FWD, 4)
ROW_CFG_MULTI(K_SM_FWD_M, 1)
ROW_CFG_MULTI(K_SM_FWD_M, 4)

#define K_SM_BWD_R(T, N, VW, R)                                                   \
  extern "C" __global__ void __launch_bounds__(BS_OF(T))                          \
      vh_sm_bwd_t##T##_n##N##_v##VW##_r##R(SoftmaxArgs a) {                       \
    softmax_bwd_impl<T, N, VW, R>(a);                                             \
  }
#define K_SM_BWD(T, N, VW) K_SM_BWD_R(T, N, VW, 1)
#define K_SM_BWD_M(T, N, VW) K_SM_BWD_R(T, N, VW, 2)
ROW_CFG_SMALL(K_SM_BWD, 1)
ROW_CFG_SMALL(K_SM_BWD, 4)
// Two-wave teams, two rows per 256-thread workgroup: the softmax form for rows
// of 129-256 units.
K_SM_FWD(128, 2, 1)
K_SM_FWD(128, 2, 4)
K_SM_BWD(128, 2, 1)
K_SM_BWD(128, 2, 4)
ROW_CFG_MULTI(K_SM_BWD_M, 1)
ROW_CFG_MULTI(K_SM_BWD_M, 4)

extern "C" __global__ void __launch_bounds__(VH_COLR_COLS * 16) vh_col_reduce(ColReduceArgs a) {
  col_reduce_impl(a);
}

// GELU
extern "C" __global__ void __launch_bounds__(256) vh_gelu_fwd_v1(EltArgs a) { gelu_flat_impl<0, 1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_gelu_fwd_v4(EltArgs a) { gelu_flat_impl<0, 4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_gelu_gradmul_v1(EltArgs a) { gelu_flat_impl<1, 1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_gelu_gradmul_v4(EltArgs a) { gelu_flat_impl<1, 4>(a); }

#define GB_CFG(M, VW) M(1, VW) M(2, VW) M(3, VW) M(4, VW) M(6, VW) M(8, VW) M(12, VW) M(16, VW)
#define K_GB_FWD(N, VW)                                                           \
  extern "C" __global__ void __launch_bounds__(256)                               \
      vh_gelu_bias_fwd_n##N##_v##VW(GeluBiasBwdArgs a) {                          \
    gelu_bias_fwd_impl<N, VW>(a);                                                 \
  }
#define K_GB_BWD(VW)                                                                      \
  extern "C" __global__ void __launch_bounds__(256) vh_gelu_bias_bwd_tile_v##VW(GeluBiasBwdArgs a) { \
    gelu_bias_bwd_tile_impl<VW, 2>(a);                                                    \
  }
#define K_GB_FWD_TILE(VW)                                                                 \
  extern "C" __global__ void __launch_bounds__(256) vh_gelu_bias_fwd_tile_v##VW(GeluBiasBwdArgs a) { \
    gelu_bias_fwd_tile_impl<VW>(a);                                                     \
  }
GB_CFG(K_GB_FWD, 1)
GB_CFG(K_GB_FWD, 4)
K_GB_FWD_TILE(1)
K_GB_FWD_TILE(4)
K_GB_BWD(1)
K_GB_BWD(4)

// Embedding
extern "C" __global__ void __launch_bounds__(256) vh_emb_fwd_v1(EmbFwdArgs a) { emb_fwd_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_fwd_v4(EmbFwdArgs a) { emb_fwd_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_tokens(EmbTokArgs a) { emb_tokens_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_alloc(EmbAllocArgs a) { emb_alloc_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_place(EmbPlaceArgs a) { emb_place_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_rows_v1(EmbSegArgs a) { emb_rows_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_rows_v4(EmbSegArgs a) { emb_rows_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_heavy_final_v1(EmbFinalArgs a) { emb_heavy_final_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_heavy_final_v4(EmbFinalArgs a) { emb_heavy_final_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(1024) vh_emb_sort(EmbSortArgs a) { emb_sort_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_sum_v1(EmbSumArgs a) { emb_sum_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_emb_sum_v4(EmbSumArgs a) { emb_sum_impl<4>(a); }

// Rows too long for the register-held row kernels (kernels/rowwide.h).
#define K_WIDE(VW)                                                                                  \
  extern "C" __global__ void __launch_bounds__(RW_TEAM) vh_sm_fwd_wide_v##VW(SoftmaxArgs a) {       \
    sm_fwd_wide_impl<VW>(a);                                                                        \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(RW_TEAM) vh_sm_bwd_wide_v##VW(SoftmaxArgs a) {       \
    sm_bwd_wide_impl<VW>(a);                                                                        \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(RW_TEAM) vh_ln_fwd_wide_v##VW(LnFwdArgs a) {         \
    ln_fwd_wide_impl<VW>(a);                                                                        \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(RW_TEAM) vh_ln_stats_wide_v##VW(LnWideArgs a) {      \
    ln_stats_wide_impl<VW>(a);                                                                      \
  }                                                                                                 \
  extern "C" __global__ void __launch_bounds__(256) vh_ln_tile_wide_v##VW(LnWideArgs a) {           \
    ln_tile_wide_impl<VW>(a);                                                                       \
  }
K_WIDE(1)
K_WIDE(4)

// Cross-entropy
// Up to NV = 104 (V <= 53,248) the kernels are held to 128 VGPRs: 4 waves per
// SIMD, two 512-thread rows per CU, one's HBM traffic overlapping the other's
// reductions. NV = 99 is the GPT-2 vocabulary (V = 50,257) exactly.
#define XE_CFG(M) M(8, 4) M(16, 4) M(24, 4) M(32, 4) M(40, 4) M(48, 4) M(56, 4) M(64, 4) M(72, 4) M(80, 4) \
  M(88, 4) M(96, 4) M(99, 4) M(104, 4) M(112, 1) M(120, 1) M(128, 1)
#define K_XE(N, W)                                                                       \
  extern "C" __global__ void __launch_bounds__(XE_TEAM, W) vh_xent_fwd_n##N(XentArgs a) { \
    xent_cached_impl<N, 0>(a);                                                           \
  }                                                                                      \
  extern "C" __global__ void __launch_bounds__(XE_TEAM, W) vh_xent_bwd_n##N(XentArgs a) { \
    xent_cached_impl<N, 1>(a);                                                           \
  }                                                                                      \
  extern "C" __global__ void __launch_bounds__(XE_TEAM, W) vh_xent_fb_n##N(XentArgs a) {  \
    xent_cached_impl<N, 2>(a);                                                           \
  }
XE_CFG(K_XE)
extern "C" __global__ void __launch_bounds__(1024) vh_xent_fwd_stream(XentArgs a) { xent_stream_impl<false>(a); }
extern "C" __global__ void __launch_bounds__(1024) vh_xent_bwd_stream(XentArgs a) { xent_stream_impl<true>(a); }
extern "C" __global__ void __launch_bounds__(1024) vh_xent_reduce(XentReduceArgs a) { xent_reduce_impl(a); }
extern "C" __global__ void __launch_bounds__(XR4_THREADS) vh_xent_bwd_rs4(XentArgs a) { xent_bwd_rs4_impl(a); }
extern "C" __global__ void __launch_bounds__(XR_THREADS) vh_xent_bwd_rs(XentArgs a) { xent_bwd_rs_impl(a); }

// Generic building blocks
extern "C" __global__ void __launch_bounds__(256) vh_binary_contig_v1(BinaryArgs a) { binary_contig_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_contig_v4(BinaryArgs a) { binary_contig_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_rowbcast_v1(BinaryArgs a) { binary_rowbcast_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_rowbcast_v4(BinaryArgs a) { binary_rowbcast_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_colbcast_v1(BinaryArgs a) { binary_colbcast_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_colbcast_v4(BinaryArgs a) { binary_colbcast_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_strided_i32(BinaryArgs a) { binary_strided_impl<uint32_t>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_binary_strided_i64(BinaryArgs a) { binary_strided_impl<uint64_t>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_reduce_thread(ReduceArgs a) { reduce_thread_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_reduce_wave(ReduceArgs a) { reduce_wave_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_strided_copy_i32(CopyArgs a) { strided_copy_impl<uint32_t>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_strided_copy_i64(CopyArgs a) { strided_copy_impl<uint64_t>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_transpose(TransposeArgs a) { transpose_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_transpose_v4(TransposeArgs a) { transpose4_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_attn_probe(AttnProbeArgs a) { attn_probe_impl(a); }
extern "C" __global__ void __launch_bounds__(64) vh_attn_decide(AttnDecideArgs a) { attn_decide_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_fill(FillArgs a) { fill_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_math_probe(MathProbeArgs a) { math_probe_impl(a); }
extern "C" __global__ void __launch_bounds__(256) vh_stream_copy(StreamCopyArgs a) { stream_copy_impl(a); }

// Matrix multiply: vh_gemm_<A><B>, each operand k-contiguous ("k") or
// m/n-contiguous ("m"/"n"), with 128-bit ("4") or 32-bit ("1") global loads.
#define K_GEMM(AK, AV, BK, BV, NAME)                                                            \
  extern "C" __global__ void __launch_bounds__(256, 2) NAME(GemmArgs a) {                      \
    gemm_f32_impl<AK, AV, BK, BV, 128>(a);                                                      \
  }                                                                                             \
  extern "C" __global__ void __launch_bounds__(256, 2) NAME##_t64(GemmArgs a) {                \
    gemm_f32_impl<AK, AV, BK, BV, 64>(a);                                                       \
  }
K_GEMM(true, true, true, true, vh_gemm_k4_k4)
K_GEMM(true, true, true, false, vh_gemm_k4_k1)
K_GEMM(true, true, false, true, vh_gemm_k4_n4)
K_GEMM(true, true, false, false, vh_gemm_k4_n1)
K_GEMM(true, false, true, true, vh_gemm_k1_k4)
K_GEMM(true, false, true, false, vh_gemm_k1_k1)
K_GEMM(true, false, false, true, vh_gemm_k1_n4)
K_GEMM(true, false, false, false, vh_gemm_k1_n1)
K_GEMM(false, true, true, true, vh_gemm_m4_k4)
K_GEMM(false, true, true, false, vh_gemm_m4_k1)
K_GEMM(false, true, false, true, vh_gemm_m4_n4)
K_GEMM(false, true, false, false, vh_gemm_m4_n1)
K_GEMM(false, false, true, true, vh_gemm_m1_k4)
K_GEMM(false, false, true, false, vh_gemm_m1_k1)
K_GEMM(false, false, false, true, vh_gemm_m1_n4)
K_GEMM(false, false, false, false, vh_gemm_m1_n1)
// Persistent form of the 128-bit-load layouts (batched products with short k).
#define K_GEMMP(AK, BK, NAME) \
  extern "C" __global__ void __launch_bounds__(256, 2) NAME(GemmArgs a) { gemm_f32_persist<AK, true, BK, true>(a); }
K_GEMMP(true, true, vh_gemmp_k4_k4)
K_GEMMP(true, false, vh_gemmp_k4_n4)
K_GEMMP(false, true, vh_gemmp_m4_k4)
K_GEMMP(false, false, vh_gemmp_m4_n4)

extern "C" __global__ void __launch_bounds__(256) vh_gemm_reduce(GemmReduceArgs a) { gemm_reduce_impl(a); }

// Large dense products: vh_gemmb_<A><B>_<BN>, persistent 256 x BN tiles (one
// 512-thread workgroup per CU), and the fix-up of its stream-K round. BN = 256
// for long k loops over a row-contiguous B (the lm_head dW products), 192
// otherwise.
#define K_GEMMB(AK, BK, BN, NAME) \
  extern "C" __global__ void __launch_bounds__(512, 1) NAME(GemmArgs a) { gemm_big_impl<AK, BK, BN, 8>(a); }
K_GEMMB(true, true, 192, vh_gemmb_kk_192)
K_GEMMB(true, false, 192, vh_gemmb_kn_192)
K_GEMMB(false, true, 192, vh_gemmb_mk_192)
K_GEMMB(false, false, 192, vh_gemmb_mn_192)
K_GEMMB(true, true, 256, vh_gemmb_kk_256)
K_GEMMB(true, false, 256, vh_gemmb_kn_256)
K_GEMMB(false, true, 256, vh_gemmb_mk_256)
K_GEMMB(false, false, 256, vh_gemmb_mn_256)
extern "C" __global__ void __launch_bounds__(256) vh_gemmb_fix_192(GemmArgs a) { gemm_big_fix_impl<192>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_gemmb_fix_256(GemmArgs a) { gemm_big_fix_impl<256>(a); }

// AdamW
extern "C" __global__ void __launch_bounds__(256) vh_adamw_v1(AdamArgs a) { adamw_impl<1>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_adamw_v4(AdamArgs a) { adamw_impl<4>(a); }
extern "C" __global__ void __launch_bounds__(256) vh_adamw_multi(AdamMultiArgs a) { adamw_multi_impl(a); }

// Row sums (bias gradients): first stage; the second is vh_col_reduce.
extern "C" __global__ void __launch_bounds__(256) vh_col_partial(ColPartialArgs a) { col_partial_impl(a); }
