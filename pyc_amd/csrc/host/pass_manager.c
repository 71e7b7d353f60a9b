/* pass_manager.c — compile-time pass pipeline over the op array.
 *
 * Behaviour of reference src/compiler/passes/pass_manager.c:
 *   canonicalize  unnamed ops become "op_<i>" (:161-170);
 *   shapes        OUTPUT/ADD/RELU/GELU/LAYERNORM copy input 0's shape and dtype,
 *                 MATMUL infers [M,N] from [M,K]x[K,N] (:172-204); CONV2D and
 *                 ATTENTION (appended kinds) infer NPQK / the query shape;
 *   fusion        MATMUL directly followed by its ADD or activation consumer is
 *                 renamed "fused_<mm>_<next>" and the consumer removed (:241-267);
 *   liveness      peak simultaneously-live values (:269-300);
 *   graph breaks  counts of kinds the compiler-next path does not lower, first
 *                 offender, compilability score and summary string (:302-393);
 *   speculation   input-size bucket, signature and confidence (:37-158).
 * The fusion output is byte-identical to the reference golden file
 * tests/compiler_next/golden/simple_pipeline_after.txt. Note that fusion drops
 * the ADD/activation semantics (as the reference's does); the engine therefore
 * never executes a fused module, it runs fusion only as analysis. */
#include "pyc/pass_manager.h"

#include <stdio.h>
#include <string.h>

static size_t elem_bytes(pyc_dtype t) {
    switch (t) {
        case PYC_DTYPE_F16:
        case PYC_DTYPE_BF16:
            return 2;
        case PYC_DTYPE_I8:
        case PYC_DTYPE_FP8_E4M3:
            return 1;
        case PYC_DTYPE_F32:
        case PYC_DTYPE_I32:
            return 4;
        default:
            return 0;
    }
}

static size_t elems(const pyc_shape* s) {
    size_t i, n = 1;
    if (!s || s->rank == 0) {
        return 0;
    }
    for (i = 0; i < s->rank; ++i) {
        if (s->dims[i] <= 0) {
            return 0;
        }
        n *= (size_t)s->dims[i];
    }
    return n;
}

static int is_act(pyc_ir_op_kind k) {
    return k == PYC_IR_OP_RELU || k == PYC_IR_OP_GELU;
}

static void pass_canonicalize(pyc_ir_module* m, pyc_pass_report* rep) {
    size_t i;
    for (i = 0; i < m->op_count; ++i) {
        if (m->ops[i].name[0] == '\0') {
            snprintf(m->ops[i].name, sizeof(m->ops[i].name), "op_%zu", i);
            rep->transformed_ops++;
        }
    }
}

static void conv_attrs(const char* name, int* sh, int* sw, int* ph, int* pw) {
    const char* at = strchr(name, '@');
    *sh = *sw = 1;
    *ph = *pw = 0;
    if (at) {
        int a, b, c, d;
        if (sscanf(at, "@s%dx%dp%dx%d", &a, &b, &c, &d) == 4) {
            *sh = a;
            *sw = b;
            *ph = c;
            *pw = d;
        }
    }
}

static int pass_shapes(pyc_ir_module* m, pyc_pass_report* rep) {
    size_t i;
    for (i = 0; i < m->op_count; ++i) {
        pyc_ir_op* op = &m->ops[i];
        switch (op->kind) {
            case PYC_IR_OP_OUTPUT:
            case PYC_IR_OP_ADD:
            case PYC_IR_OP_RELU:
            case PYC_IR_OP_GELU:
            case PYC_IR_OP_LAYERNORM:
                if (op->input_count >= 1) {
                    const pyc_ir_op* src = &m->ops[op->input_ids[0]];
                    op->shape = src->shape;
                    op->dtype = src->dtype;
                    rep->inferred_shapes++;
                }
                break;
            case PYC_IR_OP_MATMUL: {
                const pyc_ir_op *a, *b;
                if (op->input_count < 2) {
                    rep->errors++;
                    return -1;
                }
                a = &m->ops[op->input_ids[0]];
                b = &m->ops[op->input_ids[1]];
                if (a->shape.rank != 2 || b->shape.rank != 2) {
                    rep->errors++;
                    return -1;
                }
                if (b->dtype == PYC_DTYPE_FP8_E4M3) {
                    /* fp8 weight stored [N,K]: contracts dim 1 with dim 1 */
                    if (a->shape.dims[1] != b->shape.dims[1]) {
                        rep->errors++;
                        return -1;
                    }
                    op->shape.rank = 2;
                    op->shape.dims[0] = a->shape.dims[0];
                    op->shape.dims[1] = b->shape.dims[0];
                    op->dtype = a->dtype;
                } else {
                    if (a->shape.dims[1] != b->shape.dims[0]) {
                        rep->errors++;
                        return -1;
                    }
                    op->shape.rank = 2;
                    op->shape.dims[0] = a->shape.dims[0];
                    op->shape.dims[1] = b->shape.dims[1];
                    op->dtype = a->dtype;
                }
                rep->inferred_shapes++;
                break;
            }
            case PYC_IR_OP_CONV2D: {
                const pyc_ir_op *x, *w;
                int sh, sw, ph, pw;
                if (op->input_count < 2) {
                    rep->errors++;
                    return -1;
                }
                x = &m->ops[op->input_ids[0]];
                w = &m->ops[op->input_ids[1]];
                conv_attrs(op->name, &sh, &sw, &ph, &pw);
                if (x->shape.rank != 4 || w->shape.rank != 4 || x->shape.dims[3] != w->shape.dims[3] || sh <= 0 ||
                    sw <= 0 || x->shape.dims[1] + 2 * ph < w->shape.dims[1] ||
                    x->shape.dims[2] + 2 * pw < w->shape.dims[2]) {
                    rep->errors++;
                    return -1;
                }
                op->shape.rank = 4;
                op->shape.dims[0] = x->shape.dims[0];
                op->shape.dims[1] = (x->shape.dims[1] + 2 * ph - w->shape.dims[1]) / sh + 1;
                op->shape.dims[2] = (x->shape.dims[2] + 2 * pw - w->shape.dims[2]) / sw + 1;
                op->shape.dims[3] = w->shape.dims[0];
                op->dtype = x->dtype;
                rep->inferred_shapes++;
                break;
            }
            case PYC_IR_OP_ATTENTION:
                if (op->input_count < 3) {
                    rep->errors++;
                    return -1;
                }
                op->shape = m->ops[op->input_ids[0]].shape;
                op->dtype = m->ops[op->input_ids[0]].dtype;
                rep->inferred_shapes++;
                break;
            default:
                break;
        }
    }
    return 0;
}

static void drop_op(pyc_ir_module* m, size_t at) {
    size_t i, j;
    memmove(&m->ops[at], &m->ops[at + 1], (m->op_count - at - 1) * sizeof(pyc_ir_op));
    m->op_count--;
    for (i = 0; i < m->op_count; ++i) {
        for (j = 0; j < m->ops[i].input_count; ++j) {
            if ((size_t)m->ops[i].input_ids[j] > at) {
                m->ops[i].input_ids[j]--;
            }
        }
    }
}

static void pass_fuse(pyc_ir_module* m, pyc_pass_report* rep) {
    size_t i = 0;
    while (i + 1 < m->op_count) {
        pyc_ir_op* cur = &m->ops[i];
        const pyc_ir_op* nxt = &m->ops[i + 1];
        const int fusable = cur->kind == PYC_IR_OP_MATMUL &&
                            (nxt->kind == PYC_IR_OP_ADD || is_act(nxt->kind)) && nxt->input_count >= 1 &&
                            nxt->input_ids[0] == (int)i;
        if (fusable) {
            char name[PYC_IR_MAX_NAME];
            size_t k, j;
            snprintf(name, sizeof(name), "fused_%s_%s", cur->name, nxt->name);
            memcpy(cur->name, name, sizeof(cur->name));
            cur->name[sizeof(cur->name) - 1] = '\0';
            for (k = 0; k < m->op_count; ++k) {
                for (j = 0; j < m->ops[k].input_count; ++j) {
                    if (m->ops[k].input_ids[j] == (int)(i + 1)) {
                        m->ops[k].input_ids[j] = (int)i;
                    }
                }
            }
            drop_op(m, i + 1);
            rep->fused_patterns++;
            rep->transformed_ops++;
            continue;
        }
        i++;
    }
}

static void pass_liveness(const pyc_ir_module* m, pyc_pass_report* rep) {
    int last[PYC_IR_MAX_OPS];
    size_t i, j, live = 0, peak = 0;
    for (i = 0; i < m->op_count; ++i) {
        last[i] = -1;
    }
    for (i = 0; i < m->op_count; ++i) {
        for (j = 0; j < m->ops[i].input_count; ++j) {
            const int id = m->ops[i].input_ids[j];
            if (id >= 0 && (size_t)id < m->op_count) {
                last[id] = (int)i;
            }
        }
    }
    for (i = 0; i < m->op_count; ++i) {
        live++;
        if (live > peak) {
            peak = live;
        }
        if ((last[i] == (int)i || last[i] == -1) && live > 0) {
            live--;
        }
    }
    rep->peak_live_values = peak;
}

/* Kinds the compiler-next run path lowers natively. The MI355X backend adds
 * CONV2D and ATTENTION to the reference's list (pass_manager.c:302-308). */
static int lowered_kind(pyc_ir_op_kind k) {
    return k == PYC_IR_OP_INPUT || k == PYC_IR_OP_MATMUL || k == PYC_IR_OP_ADD || k == PYC_IR_OP_RELU ||
           k == PYC_IR_OP_OUTPUT || k == PYC_IR_OP_CONV2D || k == PYC_IR_OP_ATTENTION;
}

static void pass_graph_breaks(const pyc_ir_module* m, pyc_pass_report* rep) {
    size_t i, n_break = 0, counts[5] = {0, 0, 0, 0, 0};
    const char* first_reason = "none";
    const char* first_name = "none";
    int first_id = -1;
    for (i = 0; i < m->op_count; ++i) {
        const pyc_ir_op* op = &m->ops[i];
        const char* why;
        int slot;
        if (lowered_kind(op->kind)) {
            continue;
        }
        n_break++;
        switch (op->kind) {
            case PYC_IR_OP_CONST: slot = 0; why = "const"; break;
            case PYC_IR_OP_GELU: slot = 1; why = "gelu"; break;
            case PYC_IR_OP_REDUCE_SUM: slot = 2; why = "reduce_sum"; break;
            case PYC_IR_OP_LAYERNORM: slot = 3; why = "layernorm"; break;
            default: slot = 4; why = "unknown"; break;
        }
        counts[slot]++;
        if (first_id < 0) {
            first_id = (int)i;
            first_reason = why;
            first_name = op->name[0] ? op->name : "unnamed";
        }
    }
    rep->graph_break_count = n_break;
    rep->graph_break_const_count = counts[0];
    rep->graph_break_gelu_count = counts[1];
    rep->graph_break_reduce_sum_count = counts[2];
    rep->graph_break_layernorm_count = counts[3];
    rep->graph_break_unknown_count = counts[4];
    rep->first_graph_break_op_id = first_id;
    snprintf(rep->first_graph_break_op_name, sizeof(rep->first_graph_break_op_name), "%s", first_name);
    rep->compilability_score = m->op_count ? (double)(m->op_count - n_break) / (double)m->op_count : 0.0;
    snprintf(rep->graph_break_summary, sizeof(rep->graph_break_summary),
             "breaks=%zu first=%s@%d c=%zu g=%zu r=%zu l=%zu u=%zu", n_break, first_reason, first_id, counts[0],
             counts[1], counts[2], counts[3], counts[4]);
}

static void size_bucket(size_t bytes, size_t n_inputs, char* out, size_t cap) {
    const char* klass = "unknown";
    if (bytes > 0 && bytes <= 256) {
        klass = "tiny";
    } else if (bytes <= 4096) {
        klass = "small";
    } else if (bytes <= 65536) {
        klass = "medium";
    } else {
        klass = "large";
    }
    snprintf(out, cap, "%s:i%zu:b%zu", klass, n_inputs, bytes);
}

static void pass_speculation(const pyc_ir_module* m, pyc_pass_report* rep) {
    size_t i, n_in = 0, bytes = 0, used = 0;
    double conf;
    int ok = 1;
    for (i = 0; i < m->op_count; ++i) {
        if (m->ops[i].kind == PYC_IR_OP_INPUT) {
            n_in++;
            bytes += elems(&m->ops[i].shape) * elem_bytes(m->ops[i].dtype);
        }
    }
    size_bucket(bytes, n_in, rep->speculative_shape_bucket, sizeof(rep->speculative_shape_bucket));
    size_bucket(bytes, n_in, rep->phantom_shape_bucket, sizeof(rep->phantom_shape_bucket));
    rep->phantom_shape_signature[0] = '\0';
    for (i = 0; i < m->op_count && ok; ++i) {
        const pyc_ir_op* op = &m->ops[i];
        const size_t cap = sizeof(rep->phantom_shape_signature);
        size_t d;
        int n;
        if (op->kind != PYC_IR_OP_INPUT) {
            continue;
        }
        n = snprintf(rep->phantom_shape_signature + used, cap - used, "%s%d:r%zu", used ? ";" : "", (int)op->dtype,
                     op->shape.rank);
        ok = n >= 0 && (size_t)n < cap - used;
        used += ok ? (size_t)n : 0;
        for (d = 0; ok && d < op->shape.rank; ++d) {
            n = snprintf(rep->phantom_shape_signature + used, cap - used, "x%lld", (long long)op->shape.dims[d]);
            ok = n >= 0 && (size_t)n < cap - used;
            used += ok ? (size_t)n : 0;
        }
    }
    if (!ok) {
        rep->phantom_shape_signature[0] = '\0';
    }
    conf = rep->compilability_score;
    if (rep->graph_break_count > 0) {
        conf *= 0.65;
    }
    if (rep->peak_live_values > 8) {
        conf *= 0.95;
    }
    conf = conf < 0.0 ? 0.0 : (conf > 1.0 ? 1.0 : conf);
    rep->speculative_confidence = conf;
    rep->phantom_confidence = conf;
    rep->speculative_plan_count = rep->graph_break_count == 0 ? 3 : (rep->compilability_score >= 0.75 ? 2 : 1);
}

void pyc_pass_pipeline_default(pyc_pass_pipeline* p) {
    if (!p) {
        return;
    }
    memset(p, 0, sizeof(*p));
    p->config.canonicalize = 1;
    p->config.shape_inference = 1;
    p->config.layout_propagation = 1;
    p->config.fusion = 1;
    p->config.liveness = 1;
    p->config.allocation = 1;
    p->config.lowering = 1;
}

int pyc_pass_pipeline_run(pyc_pass_pipeline* p, pyc_ir_module* m, pyc_pass_report* rep) {
    if (!p || !m || !rep) {
        return -1;
    }
    memset(rep, 0, sizeof(*rep));
    if (m->op_count == 0) {
        rep->errors = 1;
        return -1;
    }
    if (p->config.canonicalize) {
        pass_canonicalize(m, rep);
        rep->passes_run++;
    }
    if (p->config.shape_inference) {
        if (pass_shapes(m, rep) != 0) {
            return -1;
        }
        rep->passes_run++;
    }
    rep->passes_run += p->config.layout_propagation ? 1 : 0; /* layouts are fixed: row-major / NHWC */
    if (p->config.fusion) {
        pass_fuse(m, rep);
        rep->passes_run++;
    }
    if (p->config.liveness) {
        pass_liveness(m, rep);
        rep->passes_run++;
    }
    rep->passes_run += p->config.allocation ? 1 : 0; /* the allocator plan is built by the engine */
    rep->passes_run += p->config.lowering ? 1 : 0;   /* lowering to device steps happens in the backend */
    pass_graph_breaks(m, rep);
    pass_speculation(m, rep);
    return 0;
}
