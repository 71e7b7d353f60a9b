/* ir.c — the bounded op-array IR: init / append / verify / text serialisation.
 *
 * Behaviour of reference src/compiler/ir/ir.c:37-170. The serialisation format
 *   "<i>:<kind>:<name>:dtype=<d>:shape=<d0>x<d1>..:inputs=<a>,<b>\n"
 * is kept byte for byte: it is the input of the model fingerprint and of the
 * reference's golden pass test (tests/compiler_next/golden/simple_pipeline_after.txt).
 * The two appended op kinds serialise as "conv2d" and "attention". */
#include "pyc/ir.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

void pyc_ir_module_init(pyc_ir_module* module) {
    if (module) {
        memset(module, 0, sizeof(*module));
    }
}

int pyc_ir_add_op(pyc_ir_module* module, const pyc_ir_op* op) {
    if (!module || !op || module->op_count >= PYC_IR_MAX_OPS) {
        return -1;
    }
    module->ops[module->op_count++] = *op;
    return 0;
}

static int fail(pyc_ir_diagnostic* diag, int code, const char* fmt, ...) {
    if (diag) {
        va_list ap;
        diag->code = code;
        va_start(ap, fmt);
        vsnprintf(diag->message, sizeof(diag->message), fmt, ap);
        va_end(ap);
    }
    return -1;
}

int pyc_ir_verify(const pyc_ir_module* module, pyc_ir_diagnostic* diag) {
    size_t i, j, d;
    if (diag) {
        memset(diag, 0, sizeof(*diag));
    }
    if (!module) {
        return fail(diag, 1, "module is NULL");
    }
    if (module->op_count == 0) {
        return fail(diag, 2, "module has no ops");
    }
    for (i = 0; i < module->op_count; ++i) {
        const pyc_ir_op* op = &module->ops[i];
        if (op->input_count > PYC_IR_MAX_INPUTS) {
            return fail(diag, 3, "op %zu has too many inputs", i);
        }
        if (op->shape.rank > PYC_IR_MAX_DIMS) {
            return fail(diag, 4, "op %zu has invalid shape", i);
        }
        for (d = 0; d < op->shape.rank; ++d) {
            if (op->shape.dims[d] <= 0) {
                return fail(diag, 4, "op %zu has invalid shape", i);
            }
        }
        for (j = 0; j < op->input_count; ++j) {
            const int id = op->input_ids[j];
            if (id < 0 || (size_t)id >= i) {
                return fail(diag, 5, "op %zu has invalid input id %d", i, id);
            }
        }
    }
    return 0;
}

static const char* op_kind_text(pyc_ir_op_kind kind) {
    static const char* const names[] = {"input", "const", "matmul", "add", "relu", "gelu",
                                        "reduce_sum", "layernorm", "output", "conv2d", "attention"};
    if ((int)kind < 0 || (int)kind > (int)PYC_IR_OP_ATTENTION) {
        return "unknown";
    }
    return names[kind];
}

/* Appends to buf at *used; returns -1 when the text does not fit. */
static int put(char* buf, size_t cap, size_t* used, const char* fmt, ...) {
    va_list ap;
    int n;
    va_start(ap, fmt);
    n = vsnprintf(buf + *used, cap - *used, fmt, ap);
    va_end(ap);
    if (n < 0 || (size_t)n >= cap - *used) {
        return -1;
    }
    *used += (size_t)n;
    return 0;
}

int pyc_ir_serialize(const pyc_ir_module* module, char* buffer, size_t buffer_size) {
    size_t i, d, used = 0;
    if (!module || !buffer || buffer_size == 0) {
        return -1;
    }
    buffer[0] = '\0';
    for (i = 0; i < module->op_count; ++i) {
        const pyc_ir_op* op = &module->ops[i];
        if (put(buffer, buffer_size, &used, "%zu:%s:%s:dtype=%d:shape=", i, op_kind_text(op->kind), op->name,
                (int)op->dtype) != 0) {
            return -1;
        }
        for (d = 0; d < op->shape.rank; ++d) {
            if (put(buffer, buffer_size, &used, d ? "x%lld" : "%lld", (long long)op->shape.dims[d]) != 0) {
                return -1;
            }
        }
        if (put(buffer, buffer_size, &used, ":inputs=") != 0) {
            return -1;
        }
        for (d = 0; d < op->input_count; ++d) {
            if (put(buffer, buffer_size, &used, d ? ",%d" : "%d", op->input_ids[d]) != 0) {
                return -1;
            }
        }
        if (put(buffer, buffer_size, &used, "\n") != 0) {
            return -1;
        }
    }
    return 0;
}
