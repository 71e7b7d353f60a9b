/* cpu_ops.h — host fp32 ops of the engine's CPU executor (cpu_ops.c). */
#ifndef PYC_CPU_OPS_H
#define PYC_CPU_OPS_H

#include <stddef.h>
#include <stdint.h>

#include "pyc/ir.h"

float pyc_cpu_bf16_to_f32(uint16_t h);
uint16_t pyc_cpu_f32_to_bf16(float f);
float pyc_cpu_f16_to_f32(uint16_t h);
uint16_t pyc_cpu_f32_to_f16(float f);
float pyc_cpu_e4m3_to_f32(uint8_t v);
/* f rounded to dtype t (bf16 / f16) and back; unchanged for other types */
float pyc_cpu_round_to(pyc_dtype t, float f);
/* threads for `work_items` independent items: PYC_NUM_THREADS (default 1, <= 32) */
int pyc_cpu_threads(size_t work_items);

/* Op attributes carried in IR op names (the reference op struct has no
 * attribute fields): CONV2D "@s<sh>x<sw>p<ph>x<pw>" (default stride 1, pad
 * 0), ATTENTION causal when the name contains "causal", LAYERNORM epsilon
 * "@eps<value>" (default 1e-5). */
void pyc_op_conv_attrs(const char* name, int* sh, int* sw, int* ph, int* pw);
int pyc_op_is_causal(const char* name);
float pyc_op_eps(const char* name);

void pyc_cpu_conv2d_nhwc(const float* x, const float* w, float* y, int N, int H, int W, int C, int K, int R, int S,
                         int ph, int pw, int sh, int sw);
/* 0, or -1 when its scratch rows cannot be allocated (o is then not written) */
int pyc_cpu_attention(const float* q, const float* k, const float* v, float* o, int B, int H, int S, int D,
                      int causal, float scale);
void pyc_cpu_w8a16_gemm(const float* x, const uint8_t* wq, const float* scale, float* y, int M, int N, int K);
void pyc_cpu_gelu(const float* x, float* y, size_t n);
void pyc_cpu_layernorm(const float* x, const float* gamma, const float* beta, float* y, size_t rows, size_t D,
                       float eps);

#endif
