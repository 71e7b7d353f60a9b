/* pyc/ir.h — bounded op-array IR consumed by the engine and the HIP backend.
 *
 * ABI mirror of the reference's IR (reference include/pyc/ir.h:1-70): the
 * struct layouts and the first enumerators keep their values so modules built
 * by a reference caller run unchanged. Append-only additions for the MI355X
 * backend: PYC_DTYPE_FP8_E4M3 (OCP e4m3fn weight storage), and the op kinds
 * PYC_IR_OP_CONV2D / PYC_IR_OP_ATTENTION so the NHWC convolution and the fused
 * causal attention are reachable from pyc_run_model. */
#ifndef PYC_IR_H
#define PYC_IR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PYC_IR_MAX_DIMS 8
#define PYC_IR_MAX_OPS 1024
#define PYC_IR_MAX_INPUTS 8
#define PYC_IR_MAX_NAME 64

/* reference include/pyc/ir.h:16-23 (values 0..5 unchanged) */
typedef enum {
    PYC_DTYPE_UNKNOWN = 0,
    PYC_DTYPE_F32 = 1,
    PYC_DTYPE_F16 = 2,
    PYC_DTYPE_BF16 = 3,
    PYC_DTYPE_I32 = 4,
    PYC_DTYPE_I8 = 5,
    PYC_DTYPE_FP8_E4M3 = 6 /* appended: OCP FP8 e4m3fn (bias 7, max 448, no inf) */
} pyc_dtype;

typedef struct {
    size_t rank;
    int64_t dims[PYC_IR_MAX_DIMS];
} pyc_shape;

/* reference include/pyc/ir.h:30-40 (values 0..8 unchanged) */
typedef enum {
    PYC_IR_OP_INPUT = 0,
    PYC_IR_OP_CONST = 1,
    PYC_IR_OP_MATMUL = 2,
    PYC_IR_OP_ADD = 3,
    PYC_IR_OP_RELU = 4,
    PYC_IR_OP_GELU = 5,
    PYC_IR_OP_REDUCE_SUM = 6,
    PYC_IR_OP_LAYERNORM = 7,
    PYC_IR_OP_OUTPUT = 8,
    /* appended: NHWC fprop convolution. inputs (x[N,H,W,C], w[K,R,S,C]);
     * output [N,P,Q,K]; stride/pad are read from the op's name suffix
     * "@s<sh>x<sw>p<ph>x<pw>" (default stride 1, pad 0). */
    PYC_IR_OP_CONV2D = 9,
    /* appended: scaled-dot-product attention. inputs (Q,K,V) [B,H,S,D];
     * causal when the op's name contains "causal"; scale 1/sqrt(D). */
    PYC_IR_OP_ATTENTION = 10
} pyc_ir_op_kind;

typedef struct {
    pyc_ir_op_kind kind;
    char name[PYC_IR_MAX_NAME];
    pyc_dtype dtype;
    pyc_shape shape;
    int input_ids[PYC_IR_MAX_INPUTS];
    size_t input_count;
} pyc_ir_op;

typedef struct {
    pyc_ir_op ops[PYC_IR_MAX_OPS];
    size_t op_count;
} pyc_ir_module;

typedef struct {
    int code;
    char message[256];
} pyc_ir_diagnostic;

/* reference include/pyc/ir.h:61-64 */
void pyc_ir_module_init(pyc_ir_module* module);
int pyc_ir_add_op(pyc_ir_module* module, const pyc_ir_op* op);
int pyc_ir_verify(const pyc_ir_module* module, pyc_ir_diagnostic* diag);
int pyc_ir_serialize(const pyc_ir_module* module, char* buffer, size_t buffer_size);

#ifdef __cplusplus
}
#endif

#endif
