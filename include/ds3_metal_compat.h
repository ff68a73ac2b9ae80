/*
 * ds3_metal_compat.h -- source-level drop-in of the ds3_hip backend for code
 * written against the reference's Metal backend (reference src/ds3_metal.h).
 *
 * Include this instead of ds3_metal.h: every ds3_metal_* name the MoE path
 * uses maps onto its ds3_hip_* counterpart, ds3_metal_buffer_t onto
 * ds3_hip_buffer_t.  ds3_type_t values pass unchanged (same GGUF ids).
 * Entry points outside the MoE path (attention, RoPE, RMSNorm, dense F32
 * matmul) are not provided by this backend.
 */
#ifndef DS3_METAL_COMPAT_H
#define DS3_METAL_COMPAT_H

#include "ds3_hip.h"

typedef ds3_hip_buffer_t ds3_metal_buffer_t;

#define ds3_metal_init ds3_hip_init
#define ds3_metal_shutdown ds3_hip_shutdown
#define ds3_metal_buffer_alloc ds3_hip_buffer_alloc
#define ds3_metal_buffer_free ds3_hip_buffer_free
#define ds3_metal_buffer_from_mmap ds3_hip_buffer_from_mmap
#define ds3_metal_buffer_view ds3_hip_buffer_view
#define ds3_metal_buffer_write ds3_hip_buffer_write
#define ds3_metal_buffer_read ds3_hip_buffer_read
#define ds3_metal_vec_matmul_f32 ds3_hip_vec_matmul_f32
#define ds3_metal_vec_matmul_quantized ds3_hip_vec_matmul_quantized
#define ds3_metal_vec_matmul_f32_simd ds3_hip_vec_matmul_f32_simd
#define ds3_metal_vec_matmul_q8_0_simd ds3_hip_vec_matmul_q8_0_simd
#define ds3_metal_vec_matmul_q4k_simd ds3_hip_vec_matmul_q4k_simd
#define ds3_metal_vec_matmul_q6k_simd ds3_hip_vec_matmul_q6k_simd
#define ds3_metal_vec_matmul_q4k_half ds3_hip_vec_matmul_q4k_half
#define ds3_metal_matmul_quantized_batch ds3_hip_matmul_quantized_batch
#define ds3_metal_buffer_copy_f32 ds3_hip_buffer_copy_f32
#define ds3_metal_buffer_zero_f32 ds3_hip_buffer_zero_f32
#define ds3_metal_vec_add_inplace ds3_hip_vec_add_inplace
#define ds3_metal_vec_add ds3_hip_vec_add
#define ds3_metal_gather_rows_f32 ds3_hip_gather_rows_f32
#define ds3_metal_scatter_add_weighted_f32 ds3_hip_scatter_add_weighted_f32
#define ds3_metal_silu_mul_f32 ds3_hip_silu_mul_f32
#define ds3_metal_rms_norm ds3_hip_rms_norm
#define ds3_metal_moe_ffn ds3_hip_moe_ffn
#define ds3_metal_moe_ffn_router ds3_hip_moe_ffn_router
#define ds3_metal_moe_ffn_experts ds3_hip_moe_ffn_experts
#define ds3_metal_moe_router_topk_batch ds3_hip_moe_router_topk_batch
#define ds3_metal_moe_router_topk_batch_tokens ds3_hip_moe_router_topk_batch_tokens
#define ds3_metal_begin_batch ds3_hip_begin_batch
#define ds3_metal_end_batch ds3_hip_end_batch
#define ds3_metal_synchronize ds3_hip_synchronize
#define ds3_metal_profile_reset ds3_hip_profile_reset
#define ds3_metal_profile_print ds3_hip_profile_print

#endif /* DS3_METAL_COMPAT_H */
