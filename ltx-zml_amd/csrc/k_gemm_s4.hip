// Small-grid GEMMs (128 x 128 tiles, four waves, two workgroups a CU):
// ltx_gemm_s4_{f16,bf16}_{i8f16,i8f32,w16}_{store,resid,qkv} for int8 weights
// with f16 or f32 scales and for 16-bit weights.
#include "gemm_s4.h"

S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f16_store, _Float16, LTX_B_I8_F16S, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f16_resid, _Float16, LTX_B_I8_F16S, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f16_qkv, _Float16, LTX_B_I8_F16S, LTX_EPI_QKV)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f32_store, _Float16, LTX_B_I8_F32S, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f32_resid, _Float16, LTX_B_I8_F32S, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_i8f32_qkv, _Float16, LTX_B_I8_F32S, LTX_EPI_QKV)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_w16_store, _Float16, LTX_B_W16, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_w16_resid, _Float16, LTX_B_W16, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_f16_w16_qkv, _Float16, LTX_B_W16, LTX_EPI_QKV)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f16_store, __bf16, LTX_B_I8_F16S, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f16_resid, __bf16, LTX_B_I8_F16S, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f16_qkv, __bf16, LTX_B_I8_F16S, LTX_EPI_QKV)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f32_store, __bf16, LTX_B_I8_F32S, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f32_resid, __bf16, LTX_B_I8_F32S, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_i8f32_qkv, __bf16, LTX_B_I8_F32S, LTX_EPI_QKV)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_w16_store, __bf16, LTX_B_W16, LTX_EPI_STORE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_w16_resid, __bf16, LTX_B_W16, LTX_EPI_RESID_GATE)
S4_GEMM_KERNEL(ltx_gemm_s4_bf16_w16_qkv, __bf16, LTX_B_W16, LTX_EPI_QKV)
