/* hip_backend.c — MI355X GPU backend behind pyc_cuda_dispatch.
 *
 * Drop-in for reference src/compiler/runtime/cuda_backend.c. It keeps:
 *   - the entry points and status codes of reference cuda_backend.h:28-98;
 *   - the dispatch order and reason vocabulary of reference
 *     cuda_backend.c:2808-2909 (forced_error, disabled_by_env,
 *     cuda_simulated_available, cuda_runtime_detected / _no_device /
 *     _error_%d, cuda_native_simulated, cuda_forced_fallback,
 *     cuda_native_unsupported_fallback, cuda_native_failed_fallback,
 *     <reason>;cpu_fallback_failed);
 *   - the env contract (PYC_CUDA_DISABLE / FORCE_ERROR / FORCE_FALLBACK /
 *     SIMULATE_AVAILABLE / ENABLE_GRAPH_REPLAY / ASSUME_STATIC_LHS|RHS /
 *     SKIP_HOST_OUTPUT_COPY / BF16_GEMM_SYMBOL / ENABLE_PROMOTED_GEMM /
 *     FORCE_HARDWARE_FAMILY); PYC_CUDA_ALLOW_TF32 / ENABLE_CUBLASLT /
 *     LT_WORKSPACE_BYTES are accepted and ignored (no TF32, no BLAS library);
 *   - one process-wide dispatch mutex (reference cuda_backend.c:13,2922-2926),
 *     a grow-only device workspace released on any native failure (:413-549,
 *     :2800-2803), static-operand upload skip (:2625-2636) and graph
 *     capture/replay of [host->device copies, kernels, device->host copies]
 *     keyed by a signature of the run (:1979-2253).
 *
 * What is new on MI355X: instead of pattern-matching one matmul[+add][+relu]
 * and running the add/relu on the host after the copy back (reference
 * cuda_backend.c:1232-1390, :1697-1742, :2783-2788), the module is lowered to a
 * list of device steps - GEMM (fp32 / bf16 / fp16 MFMA, bias and ReLU fused
 * into the epilogue), weight-only fp8 GEMM, NHWC conv (+bias +ReLU), causal
 * attention - over device buffers, one per IR value. Chains of several
 * matmuls therefore stay on the GPU and are captured into one hipGraph.
 * Reasons of successful native runs keep the reference's prefixes:
 *   hip_native_graph_capture / hip_native_graph_replay / hip_native
 * plus ":<gemm symbol>" of the first GEMM step when there is one.
 *
 * Device-resident tensors (an extension; the reference takes host pointers
 * only, compiler_api.h:83-88): a pyc_tensor whose data is device memory (by
 * hipPointerGetAttributes) is bound to the plan as it is - an input is read in
 * place, an output is written by its producing step (or by a device copy when
 * its value is an input or another output) - with no staging and no host
 * copies; host and device tensors may be mixed. Such a run waits for the
 * whole device first (the tensors may come from work on any stream), its
 * graph signature includes the device addresses, and it is never handed to
 * the simulated or CPU executor (which read host memory): a run that cannot
 * go native fails with reason "device_tensors_no_cpu_fallback". */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <math.h>

#include <hip/hip_runtime_api.h>

#include "pyc/cuda_backend.h"
#include "pyc/hip_backend.h"
#include "pyc/kernel_registry.h"
#include "cpu_ops.h"
#include "pyc_mutex.h"

/* split-K workspace of the fp8 GEMM (gemm_w8a16.hip); allocates outside capture */
int pyc_hip_w8a16_reserve(int N, int K);
/* chain kernel preconditions and its timeout word (gemm_w8a16.hip) */
int pyc_hip_w8a16_chain_supported(int M, int nsteps, const int* N, const int* K);
int pyc_hip_w8a16_chain_error_enqueue(int* host_dst, void* stream);
/* completion word of a run (run_signal.hip) */
int pyc_hip_run_signal_enqueue(uint32_t* host_word, uint32_t seq, void* stream);
/* the completion store by the run's last kernel itself (run_signal.hip) */
void pyc_hip_run_signal_arm(uint32_t* host_word, uint32_t* dev_count, uint32_t seq);
int pyc_hip_run_signal_taken(void);
/* 1 when a GEMM symbol takes alpha = 1, beta = 0 only; 1 when it names the
 * persistent kernel alone, which refuses beta != 0 and unaligned C or bias
 * (hip_kernels.c) */
int pyc_hip_gemm_symbol_unit_epilogue_only(const char* symbol);
int pyc_hip_gemm_symbol_persistent_only(const char* symbol);

static pyc_mutex g_dispatch_lock = PYC_MUTEX_INIT;

/* Measured kernel choices, filled by pyc_hip_autotune_gemm (key: dtype, M,
 * N, K) and pyc_hip_autotune_conv2d (key: dtype, N H W C K R S ph pw sh sw)
 * and read by build_plan; g_tune_gen is part of the graph signature so a new
 * choice recaptures. */
typedef struct {
    int key[12];
    char symbol[PYC_KERNEL_SYMBOL_MAX];
} tuned_entry;
#define TUNED_MAX 32
static tuned_entry g_tuned[TUNED_MAX];
static int g_tuned_count;
static tuned_entry g_tuned_conv[TUNED_MAX];
static int g_tuned_conv_count;
static uint64_t g_tune_gen;

static const char* tuned_find(const tuned_entry* tab, int count, const int* key) {
    int i;
    for (i = 0; i < count; ++i) {
        if (memcmp(tab[i].key, key, sizeof(tab[i].key)) == 0) {
            return tab[i].symbol;
        }
    }
    return NULL;
}

static const char* tuned_symbol(pyc_dtype t, int m, int n, int k) {
    int key[12] = {0};
    key[0] = (int)t;
    key[1] = m;
    key[2] = n;
    key[3] = k;
    return tuned_find(g_tuned, g_tuned_count, key);
}

static const char* tuned_conv_symbol(pyc_dtype t, const int* conv11) {
    int key[12] = {0};
    key[0] = (int)t;
    memcpy(&key[1], conv11, 11 * sizeof(int));
    return tuned_find(g_tuned_conv, g_tuned_conv_count, key);
}

/* ---------------------------------------------------------------- env */

static int env_true(const char* name) {
    const char* v = getenv(name);
    return v && (strcmp(v, "1") == 0 || strcmp(v, "true") == 0 || strcmp(v, "TRUE") == 0);
}

static int env_default_true(const char* name) {
    const char* v = getenv(name);
    if (!v || v[0] == '\0') {
        return 1;
    }
    return !(strcmp(v, "0") == 0 || strcmp(v, "false") == 0 || strcmp(v, "FALSE") == 0);
}

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec / 1e6;
}

static void set_reason(char* dst, size_t cap, const char* src) {
    if (!dst || cap == 0) {
        return;
    }
    strncpy(dst, src ? src : "", cap - 1);
    dst[cap - 1] = '\0';
}

/* ---------------------------------------------------------------- trace / family */

void pyc_cuda_dispatch_trace_init(pyc_cuda_dispatch_trace* trace) {
    if (!trace) {
        return;
    }
    memset(trace, 0, sizeof(*trace));
    set_reason(trace->reason, sizeof(trace->reason), "not_requested");
}

static pyc_mutex g_family_lock = PYC_MUTEX_INIT;
static int g_family_cached = 0;
static pyc_kernel_hardware_family g_family = PYC_KERNEL_HARDWARE_GENERIC;

pyc_kernel_hardware_family pyc_cuda_current_hardware_family(void) {
    const char* force = getenv("PYC_CUDA_FORCE_HARDWARE_FAMILY");
    pyc_kernel_hardware_family fam;
    if (force && force[0] != '\0') {
        if (strcmp(force, "cdna4") == 0 || strcmp(force, "mi355x") == 0) {
            return PYC_KERNEL_HARDWARE_CDNA4;
        }
        if (strcmp(force, "hopper") == 0) {
            return PYC_KERNEL_HARDWARE_HOPPER;
        }
        if (strcmp(force, "ada") == 0) {
            return PYC_KERNEL_HARDWARE_ADA;
        }
        if (strcmp(force, "generic") == 0) {
            return PYC_KERNEL_HARDWARE_GENERIC;
        }
    }
    pyc_mutex_lock(&g_family_lock);
    if (!g_family_cached) {
        pyc_hip_device_info info;
        g_family = PYC_KERNEL_HARDWARE_GENERIC;
        if (pyc_hip_device_query(&info) == 0 && strncmp(info.gcn_arch, "gfx950", 6) == 0) {
            g_family = PYC_KERNEL_HARDWARE_CDNA4;
        }
        g_family_cached = 1;
    }
    fam = g_family;
    pyc_mutex_unlock(&g_family_lock);
    return fam;
}

/* Number of visible devices, asked of HIP once per process (it does not
 * change while the process runs; every pyc_run_model checks it). */
static int device_count(int* count) {
    static int cached = -1;
    if (cached < 0) {
        int n = 0;
        const hipError_t err = hipGetDeviceCount(&n);
        if (err != hipSuccess) {
            return (int)err;
        }
        cached = n;
    }
    *count = cached;
    return 0;
}

static int detect_gpu(char* reason, size_t cap) {
    int count = 0;
    int err;
    if (env_true("PYC_CUDA_DISABLE")) {
        set_reason(reason, cap, "disabled_by_env");
        return 0;
    }
    if (env_true("PYC_CUDA_SIMULATE_AVAILABLE")) {
        set_reason(reason, cap, "cuda_simulated_available");
        return 1;
    }
    err = device_count(&count);
    if (err == 0 && count > 0) {
        set_reason(reason, cap, "cuda_runtime_detected");
        return 1;
    }
    if (err != 0) {
        snprintf(reason, cap, "cuda_runtime_error_%d", (int)err);
    } else {
        set_reason(reason, cap, "cuda_runtime_no_device");
    }
    return 0;
}

/* ---------------------------------------------------------------- lowering */

static size_t dtype_bytes(pyc_dtype t) {
    switch (t) {
        case PYC_DTYPE_F32:
        case PYC_DTYPE_I32:
            return 4;
        case PYC_DTYPE_F16:
        case PYC_DTYPE_BF16:
            return 2;
        case PYC_DTYPE_I8:
        case PYC_DTYPE_FP8_E4M3:
            return 1;
        default:
            return 0;
    }
}

static size_t shape_elems(const pyc_shape* s) {
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

enum { ST_GEMM = 1, ST_W8A16 = 2, ST_CONV = 3, ST_ATTN = 4, ST_GELU = 5, ST_LAYERNORM = 6 };
enum { ADD_NONE = 0, ADD_MATRIX = 1, ADD_ROW_BIAS = 2, ADD_SCALAR = 3 };

typedef struct {
    int kind;
    int out;      /* value id (op index) written */
    int in[3];    /* value ids read */
    int add_in;   /* value id of the fused add operand or -1 */
    int add_mode;
    int relu;
    pyc_dtype dtype;
    int m, n, k;  /* GEMM dims */
    int conv[11]; /* N H W C K R S ph pw sh sw */
    int attn[5];  /* B H S D causal */
    size_t elems; /* GELU: elements; LAYERNORM: rows (m) x last dim (n) */
    float eps;    /* LAYERNORM epsilon */
    int chain_len; /* fp8 steps: >= 2 on the first step of a chain launch (its length), 0 on the chain's
                    * other steps; 1 for every step that launches on its own */
    char symbol[PYC_KERNEL_SYMBOL_MAX];
} hip_step;

typedef struct {
    size_t nsteps;
    hip_step steps[PYC_IR_MAX_OPS];
    int value_op[PYC_IR_MAX_OPS];        /* op id -> op id holding its storage (fused ADD/RELU alias their producer) */
    size_t value_bytes[PYC_IR_MAX_OPS];  /* bytes of each materialised value */
    pyc_shape vshape[PYC_IR_MAX_OPS];    /* shape of each value (inferred for computed ones) */
    pyc_dtype vdtype[PYC_IR_MAX_OPS];    /* element type of each value */
    int input_ordinal[PYC_IR_MAX_OPS];   /* INPUT op -> inputs[] index, else -1 */
    int output_src[64];
    size_t n_outputs;
    int is_weight[PYC_IR_MAX_OPS];       /* INPUT read as a GEMM rhs / conv filter / fp8 scale */
    int f32_bias_needed[PYC_IR_MAX_OPS]; /* half add operand needing an fp32 device copy */
} hip_plan;

/* 1 if value v is read by no step but `reader` and is no module output. */
static int value_private(const hip_plan* p, int v, size_t reader) {
    size_t t, i;
    for (t = 0; t < p->nsteps; ++t) {
        const hip_step* st = &p->steps[t];
        if (t == reader) {
            continue;
        }
        if (st->in[0] == v || st->in[1] == v || st->in[2] == v || st->add_in == v) {
            return 0;
        }
    }
    for (i = 0; i < p->n_outputs; ++i) {
        if (p->output_src[i] == v) {
            return 0;
        }
    }
    return 1;
}

/* Number of consecutive fp8-weight steps from step s that run as one chain
 * launch (pyc_hip_w8a16_chain_dispatch): each reads the previous one's output,
 * which nothing else reads, and every step meets the chain kernel's
 * preconditions (pyc_hip_w8a16_chain_supported: K % 128 == 0 and N % 64 == 0,
 * unit and split-K slot limits; they hold step by step, so each step is
 * checked once, on its own). 1 when step s starts no chain; those steps run
 * one launch each on the per-layer kernel. build_plan stores the result in
 * each step's chain_len. */
#define HIP_CHAIN_MAX_STEPS 32
static size_t w8_chain_len(const hip_plan* p, size_t s) {
    size_t e = s;
    const hip_step* a = &p->steps[s];
    if (a->kind != ST_W8A16 || a->add_mode != ADD_NONE || !pyc_hip_w8a16_chain_supported(a->m, 1, &a->n, &a->k)) {
        return 1;
    }
    while (e + 1 < p->nsteps && e + 1 - s < HIP_CHAIN_MAX_STEPS) {
        const hip_step* cur = &p->steps[e];
        const hip_step* nx = &p->steps[e + 1];
        if (nx->kind != ST_W8A16 || nx->add_mode != ADD_NONE || nx->in[0] != cur->out || nx->m != cur->m ||
            nx->k != cur->n || !value_private(p, cur->out, e + 1) ||
            !pyc_hip_w8a16_chain_supported(nx->m, 1, &nx->n, &nx->k)) {
            break;
        }
        ++e;
    }
    return e - s + 1;
}

/* 1 when the plan launches the chain kernel somewhere. */
static int plan_has_chain(const hip_plan* p) {
    size_t s;
    for (s = 0; s < p->nsteps; ++s) {
        if (p->steps[s].chain_len >= 2) {
            return 1;
        }
    }
    return 0;
}

static int consumers(const pyc_ir_module* m, int id, int* only) {
    size_t i, j;
    int n = 0;
    for (i = 0; i < m->op_count; ++i) {
        for (j = 0; j < m->ops[i].input_count && j < PYC_IR_MAX_INPUTS; ++j) {
            if (m->ops[i].input_ids[j] == id) {
                n++;
                if (only) {
                    *only = (int)i;
                }
            }
        }
    }
    return n;
}

static int valid_id(const pyc_ir_module* m, int id) {
    return id >= 0 && (size_t)id < m->op_count;
}

static void set_value(hip_plan* plan, int id, const pyc_shape* shape, pyc_dtype t) {
    plan->vshape[id] = *shape;
    plan->vdtype[id] = t;
    plan->value_bytes[id] = shape_elems(shape) * dtype_bytes(t);
}

/* Absorb "x -> ADD(x, operand) -> RELU" after the GEMM/conv step `st` whose
 * output value `prod` is viewed as [rows, cols]. Marks the absorbed ops in
 * `covered` and makes them aliases of `prod`. */
static void absorb_epilogue(const pyc_ir_module* m, int prod, size_t rows, size_t cols, hip_step* st,
                            hip_plan* plan, int* covered) {
    int next = -1;
    int cur = prod;
    st->add_in = -1;
    st->add_mode = ADD_NONE;
    st->relu = 0;
    if (consumers(m, cur, &next) == 1 && m->ops[next].kind == PYC_IR_OP_ADD && m->ops[next].input_count >= 2) {
        const pyc_ir_op* add = &m->ops[next];
        int other = add->input_ids[0] == cur ? add->input_ids[1] : (add->input_ids[1] == cur ? add->input_ids[0] : -1);
        if (valid_id(m, other) && m->ops[other].kind == PYC_IR_OP_INPUT) {
            const pyc_shape* s = &m->ops[other].shape;
            int mode = ADD_NONE;
            if (s->rank == 2 && (size_t)s->dims[0] == rows && (size_t)s->dims[1] == cols) {
                mode = ADD_MATRIX;
            } else if (s->rank == 1 && (size_t)s->dims[0] == cols) {
                mode = ADD_ROW_BIAS;
            } else if (s->rank == 1 && s->dims[0] == 1) {
                mode = ADD_SCALAR;
            }
            if (mode != ADD_NONE && (mode != ADD_MATRIX || m->ops[other].dtype == st->dtype) &&
                (m->ops[other].dtype == PYC_DTYPE_F32 || m->ops[other].dtype == st->dtype)) {
                st->add_in = other;
                st->add_mode = mode;
                if (mode != ADD_MATRIX && m->ops[other].dtype != PYC_DTYPE_F32) {
                    plan->f32_bias_needed[other] = 1;
                }
                plan->value_op[next] = prod;
                set_value(plan, next, &plan->vshape[prod], plan->vdtype[prod]);
                covered[next] = 1;
                cur = next;
            }
        }
    }
    next = -1;
    if (consumers(m, cur, &next) == 1 && m->ops[next].kind == PYC_IR_OP_RELU) {
        st->relu = 1;
        plan->value_op[next] = prod;
        set_value(plan, next, &plan->vshape[prod], plan->vdtype[prod]);
        covered[next] = 1;
    }
}

/* The shape-chosen GEMM symbol of a dtype, which takes every shape, epilogue
 * and alignment (the planned symbol when a tuned, promoted or env-selected one
 * cannot run a step). */
static const char* general_gemm_symbol(pyc_dtype t) {
    return t == PYC_DTYPE_BF16 ? "hip_gemm_bf16_nn" : t == PYC_DTYPE_F16 ? "hip_gemm_f16_nn" : "hip_gemm_f32_nn_64x64";
}

static const char* default_gemm_symbol(pyc_dtype t) {
    if (t == PYC_DTYPE_BF16) {
        const char* env = getenv("PYC_CUDA_BF16_GEMM_SYMBOL");
        return (env && env[0] != '\0') ? env : "hip_gemm_bf16_nn";
    }
    if (t == PYC_DTYPE_F16) {
        return "hip_gemm_f16_nn";
    }
    return "hip_gemm_f32_nn_64x64";
}

/* Build the device plan; returns 0 on success, 1 when some op has no native
 * lowering (the caller then falls back). */
static int build_plan(const pyc_ir_module* m, hip_plan* plan) {
    size_t i;
    int covered[PYC_IR_MAX_OPS];
    size_t n_in = 0;
    memset(covered, 0, sizeof(covered));
    plan->nsteps = 0;
    plan->n_outputs = 0;
    for (i = 0; i < m->op_count; ++i) {
        plan->value_op[i] = (int)i;
        plan->value_bytes[i] = 0;
        memset(&plan->vshape[i], 0, sizeof(pyc_shape));
        plan->vdtype[i] = PYC_DTYPE_UNKNOWN;
        plan->input_ordinal[i] = -1;
        plan->is_weight[i] = 0;
        plan->f32_bias_needed[i] = 0;
    }
    for (i = 0; i < m->op_count; ++i) {
        const pyc_ir_op* op = &m->ops[i];
        hip_step* st = &plan->steps[plan->nsteps];
        if (covered[i]) {
            continue;
        }
        switch (op->kind) {
            case PYC_IR_OP_INPUT:
                plan->input_ordinal[i] = (int)n_in++;
                set_value(plan, (int)i, &op->shape, op->dtype);
                if (plan->value_bytes[i] == 0) {
                    return 1;
                }
                break;
            case PYC_IR_OP_MATMUL: {
                int a = op->input_count >= 2 ? op->input_ids[0] : -1;
                int b = op->input_count >= 2 ? op->input_ids[1] : -1;
                pyc_shape out_shape;
                const pyc_shape *as, *bs;
                if (!valid_id(m, a) || !valid_id(m, b) || a >= (int)i || b >= (int)i) {
                    return 1;
                }
                a = plan->value_op[a];
                b = plan->value_op[b];
                as = &plan->vshape[a];
                bs = &plan->vshape[b];
                if (as->rank != 2 || bs->rank != 2) {
                    return 1;
                }
                memset(st, 0, sizeof(*st));
                st->out = (int)i;
                st->in[0] = a;
                st->in[1] = b;
                st->in[2] = -1;
                if (plan->vdtype[b] == PYC_DTYPE_FP8_E4M3) {
                    /* weight-only fp8: rhs INPUT stored [N,K], third input = fp32 scale[N] */
                    int sc = op->input_count >= 3 ? op->input_ids[2] : -1;
                    if (!valid_id(m, sc) || m->ops[sc].kind != PYC_IR_OP_INPUT || m->ops[sc].dtype != PYC_DTYPE_F32 ||
                        m->ops[b].kind != PYC_IR_OP_INPUT || plan->vdtype[a] != PYC_DTYPE_BF16) {
                        return 1;
                    }
                    st->kind = ST_W8A16;
                    st->dtype = PYC_DTYPE_BF16;
                    st->m = (int)as->dims[0];
                    st->k = (int)as->dims[1];
                    st->n = (int)bs->dims[0];
                    if (bs->dims[1] != st->k || m->ops[sc].shape.rank != 1 || m->ops[sc].shape.dims[0] != st->n ||
                        st->m > 32 || (st->k % 16) != 0) {
                        return 1;
                    }
                    st->in[2] = sc;
                    plan->is_weight[b] = 1;
                    plan->is_weight[sc] = 1;
                    set_reason(st->symbol, sizeof(st->symbol), "hip_gemm_w8a16_e4m3");
                } else {
                    const pyc_dtype t = plan->vdtype[a];
                    if (t != PYC_DTYPE_F32 && t != PYC_DTYPE_BF16 && t != PYC_DTYPE_F16) {
                        return 1;
                    }
                    if (plan->vdtype[b] != t || (op->dtype != t && op->dtype != PYC_DTYPE_UNKNOWN)) {
                        return 1;
                    }
                    st->kind = ST_GEMM;
                    st->dtype = t;
                    st->m = (int)as->dims[0];
                    st->k = (int)as->dims[1];
                    if (bs->dims[0] != st->k) {
                        return 1;
                    }
                    st->n = (int)bs->dims[1];
                    if (m->ops[b].kind == PYC_IR_OP_INPUT) {
                        plan->is_weight[b] = 1;
                    }
                    set_reason(st->symbol, sizeof(st->symbol), default_gemm_symbol(t));
                    if (tuned_symbol(t, st->m, st->n, st->k)) {
                        set_reason(st->symbol, sizeof(st->symbol), tuned_symbol(t, st->m, st->n, st->k));
                    }
                    if (t == PYC_DTYPE_F32 && env_true("PYC_CUDA_ENABLE_PROMOTED_GEMM")) {
                        char promoted[PYC_KERNEL_SYMBOL_MAX];
                        if (pyc_kernel_promoted_symbol("matmul", PYC_BACKEND_CUDA, promoted, sizeof(promoted)) == 0 &&
                            (strcmp(promoted, "ada_gemm_k64_warp32_async_f32") == 0 ||
                             strcmp(promoted, "hip_gemm_f32_nn_64x64") == 0)) {
                            set_reason(st->symbol, sizeof(st->symbol), promoted);
                        }
                    }
                }
                memset(&out_shape, 0, sizeof(out_shape));
                out_shape.rank = 2;
                out_shape.dims[0] = st->m;
                out_shape.dims[1] = st->n;
                set_value(plan, (int)i, &out_shape, st->dtype);
                absorb_epilogue(m, (int)i, (size_t)st->m, (size_t)st->n, st, plan, covered);
                if (st->kind == ST_W8A16 && st->add_mode != ADD_NONE) {
                    return 1; /* the fp8 epilogue is scale (+ReLU) only */
                }
                if (st->kind == ST_GEMM && st->add_mode == ADD_MATRIX &&
                    (pyc_hip_gemm_symbol_unit_epilogue_only(st->symbol) ||
                     pyc_hip_gemm_symbol_persistent_only(st->symbol))) {
                    /* a matrix addend runs as beta = 1, which a tuned,
                     * promoted or env-selected unit-epilogue or
                     * persistent-only variant does not take */
                    set_reason(st->symbol, sizeof(st->symbol), general_gemm_symbol(st->dtype));
                }
                plan->nsteps++;
                break;
            }
            case PYC_IR_OP_CONV2D: {
                int x = op->input_count >= 2 ? op->input_ids[0] : -1;
                int w = op->input_count >= 2 ? op->input_ids[1] : -1;
                int sh, sw, ph, pw;
                int64_t P, Q;
                pyc_shape out_shape;
                const pyc_shape *xs, *ws;
                if (!valid_id(m, x) || !valid_id(m, w) || x >= (int)i || w >= (int)i) {
                    return 1;
                }
                x = plan->value_op[x];
                w = plan->value_op[w];
                xs = &plan->vshape[x];
                ws = &plan->vshape[w];
                if (xs->rank != 4 || ws->rank != 4 || xs->dims[3] != ws->dims[3]) {
                    return 1;
                }
                if ((plan->vdtype[x] != PYC_DTYPE_BF16 && plan->vdtype[x] != PYC_DTYPE_F16) ||
                    plan->vdtype[w] != plan->vdtype[x]) {
                    return 1;
                }
                pyc_op_conv_attrs(op->name, &sh, &sw, &ph, &pw);
                memset(st, 0, sizeof(*st));
                st->kind = ST_CONV;
                st->dtype = plan->vdtype[x];
                st->out = (int)i;
                st->in[0] = x;
                st->in[1] = w;
                st->in[2] = -1;
                st->conv[0] = (int)xs->dims[0];
                st->conv[1] = (int)xs->dims[1];
                st->conv[2] = (int)xs->dims[2];
                st->conv[3] = (int)xs->dims[3];
                st->conv[4] = (int)ws->dims[0];
                st->conv[5] = (int)ws->dims[1];
                st->conv[6] = (int)ws->dims[2];
                st->conv[7] = ph;
                st->conv[8] = pw;
                st->conv[9] = sh;
                st->conv[10] = sw;
                if (sh <= 0 || sw <= 0 || ph < 0 || pw < 0 || st->conv[1] + 2 * ph < st->conv[5] ||
                    st->conv[2] + 2 * pw < st->conv[6] || (st->conv[3] % 8) != 0) {
                    return 1;
                }
                P = (st->conv[1] + 2 * ph - st->conv[5]) / sh + 1;
                Q = (st->conv[2] + 2 * pw - st->conv[6]) / sw + 1;
                if (m->ops[w].kind == PYC_IR_OP_INPUT) {
                    plan->is_weight[w] = 1;
                }
                set_reason(st->symbol, sizeof(st->symbol),
                           st->dtype == PYC_DTYPE_BF16 ? "hip_conv2d_bf16" : "hip_conv2d_f16");
                if (tuned_conv_symbol(st->dtype, st->conv)) {
                    set_reason(st->symbol, sizeof(st->symbol), tuned_conv_symbol(st->dtype, st->conv));
                }
                memset(&out_shape, 0, sizeof(out_shape));
                out_shape.rank = 4;
                out_shape.dims[0] = st->conv[0];
                out_shape.dims[1] = P;
                out_shape.dims[2] = Q;
                out_shape.dims[3] = st->conv[4];
                set_value(plan, (int)i, &out_shape, st->dtype);
                absorb_epilogue(m, (int)i, (size_t)(st->conv[0] * P * Q), (size_t)st->conv[4], st, plan, covered);
                if (st->add_mode != ADD_NONE && st->add_mode != ADD_ROW_BIAS) {
                    return 1;
                }
                plan->nsteps++;
                break;
            }
            case PYC_IR_OP_ATTENTION: {
                int q = op->input_count >= 3 ? op->input_ids[0] : -1;
                int kk = op->input_count >= 3 ? op->input_ids[1] : -1;
                int v = op->input_count >= 3 ? op->input_ids[2] : -1;
                const pyc_shape* qs;
                if (!valid_id(m, q) || !valid_id(m, kk) || !valid_id(m, v) || q >= (int)i || kk >= (int)i ||
                    v >= (int)i) {
                    return 1;
                }
                q = plan->value_op[q];
                kk = plan->value_op[kk];
                v = plan->value_op[v];
                qs = &plan->vshape[q];
                if (qs->rank != 4 || (plan->vdtype[q] != PYC_DTYPE_BF16 && plan->vdtype[q] != PYC_DTYPE_F16)) {
                    return 1;
                }
                if (plan->vshape[kk].rank != 4 || plan->vshape[v].rank != 4 ||
                    memcmp(plan->vshape[kk].dims, qs->dims, 4 * sizeof(int64_t)) != 0 ||
                    memcmp(plan->vshape[v].dims, qs->dims, 4 * sizeof(int64_t)) != 0 ||
                    plan->vdtype[kk] != plan->vdtype[q] || plan->vdtype[v] != plan->vdtype[q]) {
                    return 1;
                }
                memset(st, 0, sizeof(*st));
                st->kind = ST_ATTN;
                st->dtype = plan->vdtype[q];
                st->out = (int)i;
                st->in[0] = q;
                st->in[1] = kk;
                st->in[2] = v;
                st->add_in = -1;
                st->attn[0] = (int)qs->dims[0];
                st->attn[1] = (int)qs->dims[1];
                st->attn[2] = (int)qs->dims[2];
                st->attn[3] = (int)qs->dims[3];
                st->attn[4] = pyc_op_is_causal(op->name);
                if (st->attn[3] != 64 && st->attn[3] != 128) {
                    return 1;
                }
                set_reason(st->symbol, sizeof(st->symbol),
                           st->dtype == PYC_DTYPE_BF16 ? "hip_attention_bf16" : "hip_attention_f16");
                set_value(plan, (int)i, qs, st->dtype);
                plan->nsteps++;
                break;
            }
            case PYC_IR_OP_GELU:
            case PYC_IR_OP_LAYERNORM: {
                /* GELU (exact erf form) elementwise; LAYERNORM over the last
                 * dimension with optional gamma (input 1) and beta (input 2)
                 * of shape [D] and x's type, epsilon 1e-5 or "@eps<value>" in
                 * the op name. The reference executes neither (its pass
                 * report counts them as graph breaks, reference
                 * src/compiler/passes/pass_manager.c:313-373). */
                const int is_ln = op->kind == PYC_IR_OP_LAYERNORM;
                int x = op->input_count >= 1 ? op->input_ids[0] : -1;
                size_t k;
                if (!valid_id(m, x) || x >= (int)i || op->input_count > (is_ln ? 3u : 1u)) {
                    return 1;
                }
                x = plan->value_op[x];
                if (plan->value_bytes[x] == 0 || (plan->vdtype[x] != PYC_DTYPE_F32 && plan->vdtype[x] != PYC_DTYPE_BF16 &&
                                                  plan->vdtype[x] != PYC_DTYPE_F16)) {
                    return 1;
                }
                memset(st, 0, sizeof(*st));
                st->kind = is_ln ? ST_LAYERNORM : ST_GELU;
                st->dtype = plan->vdtype[x];
                st->out = (int)i;
                st->in[0] = x;
                st->in[1] = st->in[2] = -1;
                st->add_in = -1;
                st->elems = shape_elems(&plan->vshape[x]);
                if (is_ln) {
                    const pyc_shape* xs = &plan->vshape[x];
                    if (xs->rank < 1 || xs->dims[xs->rank - 1] <= 0 || xs->dims[xs->rank - 1] > 0x7FFFFFFF) {
                        return 1;
                    }
                    st->n = (int)xs->dims[xs->rank - 1];
                    if (st->elems / (size_t)st->n > 0x7FFFFFFF) {
                        return 1;
                    }
                    st->m = (int)(st->elems / (size_t)st->n);
                    st->eps = pyc_op_eps(op->name);
                    if (!(st->eps >= 0.0f)) {
                        return 1;
                    }
                    for (k = 1; k < op->input_count; ++k) {
                        int gb = op->input_ids[k];
                        if (!valid_id(m, gb) || gb >= (int)i) {
                            return 1;
                        }
                        gb = plan->value_op[gb];
                        if (plan->vdtype[gb] != st->dtype || shape_elems(&plan->vshape[gb]) != (size_t)st->n) {
                            return 1;
                        }
                        st->in[k] = gb;
                    }
                }
                set_reason(st->symbol, sizeof(st->symbol),
                           st->dtype == PYC_DTYPE_F32 ? (is_ln ? "hip_layernorm_f32" : "hip_gelu_f32")
                           : st->dtype == PYC_DTYPE_BF16 ? (is_ln ? "hip_layernorm_bf16" : "hip_gelu_bf16")
                                                          : (is_ln ? "hip_layernorm_f16" : "hip_gelu_f16"));
                set_value(plan, (int)i, &plan->vshape[x], st->dtype);
                plan->nsteps++;
                break;
            }
            case PYC_IR_OP_OUTPUT: {
                int src = op->input_count >= 1 ? op->input_ids[0] : -1;
                if (!valid_id(m, src) || src >= (int)i || plan->n_outputs >= 64) {
                    return 1;
                }
                src = plan->value_op[src];
                if (plan->value_bytes[src] == 0) {
                    return 1;
                }
                plan->output_src[plan->n_outputs++] = src;
                break;
            }
            default:
                return 1; /* ADD/RELU not absorbed, CONST, REDUCE_SUM */
        }
    }
    for (i = 0; i < plan->nsteps;) {
        const size_t clen = w8_chain_len(plan, i);
        size_t j;
        plan->steps[i].chain_len = (int)clen;
        for (j = 1; j < clen; ++j) {
            plan->steps[i + j].chain_len = 0;
        }
        i += clen;
    }
    return 0;
}

/* ---------------------------------------------------------------- workspace */

typedef struct {
    void* ptr;
    size_t cap;
} dbuf;

typedef struct {
    void* ptr;
    size_t cap;
} hbuf;

/* Executable graphs kept for replay. A process that alternates models (a
 * prefill and a decode module, say) replays each one's graph instead of
 * re-capturing on every switch. */
#define GRAPH_SLOTS 8

typedef struct {
    int valid;
    uint64_t sig;
    uint64_t last_use;
    hipGraph_t graph;
    hipGraphExec_t exec;
} graph_slot;

static struct {
    int ready;
    int device;
    hipStream_t stream;
    hipEvent_t ev0, ev1;
    dbuf val[PYC_IR_MAX_OPS];      /* device storage per value (op id) */
    dbuf bias32[PYC_IR_MAX_OPS];   /* fp32 copies / fills of add operands */
    hbuf stage_in[PYC_IR_MAX_OPS]; /* pinned staging per INPUT op */
    hbuf stage_out[64];            /* pinned staging per output ordinal */
    const void* last_host[PYC_IR_MAX_OPS];
    size_t last_bytes[PYC_IR_MAX_OPS];
    int uploaded[PYC_IR_MAX_OPS];
    int* chain_err;                /* pinned copy of the chain kernel's timeout word */
    uint32_t* done_word;           /* pinned, host-coherent completion word (run_signal.hip) */
    uint32_t done_seq;             /* sequence number of the last run that signalled */
    uint32_t* done_count;          /* device arrival counter of a kernel that signals itself */
    uint64_t upload_module;        /* module whose static inputs val[] holds (uploaded[]) */
    /* graph replay: one executable graph per run signature, least recently
     * used one replaced */
    graph_slot graphs[GRAPH_SLOTS];
    uint64_t graph_clock;
} g_ws;

/* Destroys every cached graph: they bake in workspace addresses, so a buffer
 * that moves (or is released) invalidates all of them. */
static void graphs_flush(void) {
    size_t i;
    for (i = 0; i < GRAPH_SLOTS; ++i) {
        if (g_ws.graphs[i].valid) {
            (void)hipGraphExecDestroy(g_ws.graphs[i].exec);
            (void)hipGraphDestroy(g_ws.graphs[i].graph);
            g_ws.graphs[i].valid = 0;
        }
    }
}

static graph_slot* graph_find(uint64_t sig) {
    size_t i;
    for (i = 0; i < GRAPH_SLOTS; ++i) {
        if (g_ws.graphs[i].valid && g_ws.graphs[i].sig == sig) {
            g_ws.graphs[i].last_use = ++g_ws.graph_clock;
            return &g_ws.graphs[i];
        }
    }
    return NULL;
}

/* A free slot, else the least recently used one (its graph destroyed). */
static graph_slot* graph_victim(void) {
    size_t i, v = 0;
    for (i = 0; i < GRAPH_SLOTS; ++i) {
        if (!g_ws.graphs[i].valid) {
            return &g_ws.graphs[i];
        }
        if (g_ws.graphs[i].last_use < g_ws.graphs[v].last_use) {
            v = i;
        }
    }
    (void)hipGraphExecDestroy(g_ws.graphs[v].exec);
    (void)hipGraphDestroy(g_ws.graphs[v].graph);
    g_ws.graphs[v].valid = 0;
    return &g_ws.graphs[v];
}

static void ws_release(void) {
    size_t i;
    graphs_flush();
    for (i = 0; i < PYC_IR_MAX_OPS; ++i) {
        if (g_ws.val[i].ptr) {
            (void)hipFree(g_ws.val[i].ptr);
        }
        if (g_ws.bias32[i].ptr) {
            (void)hipFree(g_ws.bias32[i].ptr);
        }
        if (g_ws.stage_in[i].ptr) {
            (void)hipHostFree(g_ws.stage_in[i].ptr);
        }
    }
    for (i = 0; i < 64; ++i) {
        if (g_ws.stage_out[i].ptr) {
            (void)hipHostFree(g_ws.stage_out[i].ptr);
        }
    }
    if (g_ws.chain_err) {
        (void)hipHostFree(g_ws.chain_err);
    }
    if (g_ws.done_word) {
        (void)hipHostFree(g_ws.done_word);
    }
    if (g_ws.done_count) {
        (void)hipFree(g_ws.done_count);
    }
    if (g_ws.ready) {
        (void)hipEventDestroy(g_ws.ev0);
        (void)hipEventDestroy(g_ws.ev1);
        (void)hipStreamDestroy(g_ws.stream);
    }
    memset(&g_ws, 0, sizeof(g_ws));
}

static int ws_init(void) {
    if (g_ws.ready) {
        return 0;
    }
    memset(&g_ws, 0, sizeof(g_ws));
    if (hipGetDevice(&g_ws.device) != hipSuccess) {
        return -1;
    }
    if (hipStreamCreateWithFlags(&g_ws.stream, hipStreamNonBlocking) != hipSuccess) {
        return -1;
    }
    if (hipEventCreate(&g_ws.ev0) != hipSuccess || hipEventCreate(&g_ws.ev1) != hipSuccess) {
        return -1;
    }
    if (hipHostMalloc((void**)&g_ws.chain_err, 64, hipHostMallocDefault) != hipSuccess) {
        g_ws.chain_err = NULL;
        return -1;
    }
    *g_ws.chain_err = 0;
    if (hipHostMalloc((void**)&g_ws.done_word, 64, hipHostMallocCoherent) != hipSuccess) {
        g_ws.done_word = NULL;
        return -1;
    }
    *g_ws.done_word = 0;
    g_ws.done_seq = 0;
    /* the signalling kernels' counters: 9 x 256 bytes (run_signal_arrive) */
    if (hipMalloc((void**)&g_ws.done_count, 4096) != hipSuccess) {
        g_ws.done_count = NULL;
        return -1;
    }
    if (hipMemset(g_ws.done_count, 0, 4096) != hipSuccess) {
        return -1;
    }
    g_ws.ready = 1;
    return 0;
}

/* Waits for the run whose completion word is `seq` (run_signal.hip): spins on
 * the word for up to 2 ms, the span of the short runs whose latency the spin
 * saves, then blocks in hipStreamSynchronize, which also reports any error of
 * the stream's work. 0 when the run completed. */
static int wait_done_word(uint32_t seq) {
    const double t_start = now_ms();
    unsigned spins = 0;
    while (__atomic_load_n(g_ws.done_word, __ATOMIC_ACQUIRE) != seq) {
        if ((++spins & 255u) == 0 && now_ms() - t_start > 2.0) {
            if (hipStreamSynchronize(g_ws.stream) != hipSuccess) {
                return -1;
            }
            return __atomic_load_n(g_ws.done_word, __ATOMIC_ACQUIRE) == seq ? 0 : -1;
        }
    }
    return 0;
}

/* Grow-only device buffer; growth invalidates the captured graphs. */
static int dgrow(dbuf* b, size_t bytes) {
    if (b->cap >= bytes && b->ptr) {
        return 0;
    }
    graphs_flush();
    if (b->ptr) {
        (void)hipFree(b->ptr);
        b->ptr = NULL;
        b->cap = 0;
    }
    if (hipMalloc(&b->ptr, bytes) != hipSuccess) {
        b->ptr = NULL;
        return -1;
    }
    b->cap = bytes;
    return 0;
}

static int hgrow(hbuf* b, size_t bytes) {
    if (b->cap >= bytes && b->ptr) {
        return 0;
    }
    graphs_flush();
    if (b->ptr) {
        (void)hipHostFree(b->ptr);
        b->ptr = NULL;
        b->cap = 0;
    }
    if (hipHostMalloc(&b->ptr, bytes, hipHostMallocDefault) != hipSuccess) {
        b->ptr = NULL;
        return -1;
    }
    b->cap = bytes;
    return 0;
}

static float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    float f;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            exp = 1;
            while (!(man & 0x400u)) {
                man <<= 1;
                exp--;
            }
            man &= 0x3ffu;
            u = sign | ((uint32_t)(exp + 112) << 23) | (man << 13);
        }
    } else {
        u = sign | ((uint32_t)(exp + 112) << 23) | (man << 13);
    }
    memcpy(&f, &u, sizeof(f));
    return f;
}

/* ---------------------------------------------------------------- execution */

/* 1 when p is device (or managed) memory, 0 for host memory, pageable or
 * pinned. Tensors in device memory are bound to the plan directly: no
 * staging, no copies (the caller keeps its tensors resident). */
static int is_device_ptr(const void* p) {
    hipPointerAttribute_t a;
    if (!p) {
        return 0;
    }
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError(); /* an unregistered host pointer leaves an error behind */
        return 0;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

/* Any input or output tensor in device memory (the CPU executor cannot take them). */
static int any_device_tensor(const pyc_tensor* inputs, size_t input_count, const pyc_tensor* outputs,
                             size_t output_count) {
    size_t i;
    for (i = 0; i < input_count; ++i) {
        if (is_device_ptr(inputs[i].data)) {
            return 1;
        }
    }
    for (i = 0; i < output_count; ++i) {
        if (is_device_ptr(outputs[i].data)) {
            return 1;
        }
    }
    return 0;
}

/* Run-signature hash: FNV-1a's multiply over 8-byte words (then the tail
 * bytes), with a shift-xor so high bits reach the low ones. Only equality of
 * two signatures matters; it runs on every call, so it takes words. */
static uint64_t fnv(uint64_t h, const void* p, size_t n) {
    const unsigned char* c = (const unsigned char*)p;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, c + i, sizeof(w));
        h = (h ^ w) * 1099511628211ull;
        h ^= h >> 29;
    }
    for (; i < n; ++i) {
        h = (h ^ c[i]) * 1099511628211ull;
    }
    return h;
}

/* Enqueues the plan's kernels on the backend stream; vp[v] is the device
 * storage of value v (workspace, or the caller's device tensor). arm_seq != 0:
 * the run's last kernel is also its last work on the stream, and when that
 * kernel can store the completion word itself (the fp32 LDS-DMA GEMM) it is
 * launched so; *signalled says whether it was. */
static int enqueue_steps(const pyc_ir_module* m, const hip_plan* plan, void* const* vp, uint32_t arm_seq,
                         int* signalled, char* why, size_t why_cap) {
    size_t s;
    void* st_stream = (void*)g_ws.stream;
    *signalled = 0;
    for (s = 0; s < plan->nsteps; ++s) {
        const hip_step* st = &plan->steps[s];
        void* out = vp[st->out];
        const size_t clen = (size_t)st->chain_len;
        const int arm = arm_seq != 0 && s + 1 == plan->nsteps && st->kind == ST_GEMM;
        if (clen >= 2) {
            /* the whole run of fp8-weight steps in one launch */
            const void* wq[HIP_CHAIN_MAX_STEPS];
            const float* sc[HIP_CHAIN_MAX_STEPS];
            int cn[HIP_CHAIN_MAX_STEPS], ck[HIP_CHAIN_MAX_STEPS], cr[HIP_CHAIN_MAX_STEPS];
            size_t c;
            for (c = 0; c < clen; ++c) {
                const hip_step* q = &plan->steps[s + c];
                wq[c] = vp[q->in[1]];
                sc[c] = (const float*)vp[q->in[2]];
                cn[c] = q->n;
                ck[c] = q->k;
                cr[c] = q->relu;
            }
            if (pyc_hip_w8a16_chain_dispatch("hip_w8a16_chain_e4m3", st->m, (int)clen, vp[st->in[0]], wq,
                                             sc, cn, ck, cr, vp[plan->steps[s + clen - 1].out],
                                             st_stream) != 0) {
                snprintf(why, why_cap, "hip_kernel_failed:hip_w8a16_chain_e4m3");
                return -1;
            }
            s += clen - 1;
            continue;
        }
        int rc = -1;
        int epi = (st->relu ? PYC_HIP_EPI_RELU : 0);
        const float* bias = NULL;
        float beta = 0.0f;
        if (st->add_mode == ADD_ROW_BIAS || st->add_mode == ADD_SCALAR) {
            epi |= PYC_HIP_EPI_BIAS;
            /* an fp32 row bias is read where it was uploaded; scalar and half
             * operands use their converted fp32 copy */
            bias = (st->add_mode == ADD_ROW_BIAS && !plan->f32_bias_needed[st->add_in])
                       ? (const float*)vp[st->add_in]
                       : (const float*)g_ws.bias32[st->add_in].ptr;
        } else if (st->add_mode == ADD_MATRIX) {
            /* C starts as the addend; beta = 1 folds it into the epilogue */
            if (hipMemcpyAsync(out, vp[st->add_in], (size_t)st->m * st->n * dtype_bytes(st->dtype),
                               hipMemcpyDeviceToDevice, g_ws.stream) != hipSuccess) {
                snprintf(why, why_cap, "hip_copy_failed");
                return -1;
            }
            beta = 1.0f;
        }
        if (arm) {
            pyc_hip_run_signal_arm(g_ws.done_word, g_ws.done_count, arm_seq);
        }
        switch (st->kind) {
            case ST_GEMM:
                rc = pyc_hip_gemm_dispatch(st->symbol, st->m, st->n, st->k, vp[st->in[0]],
                                           vp[st->in[1]], out, 1.0f, beta, bias, epi, st_stream);
                if (rc == -1 && pyc_hip_gemm_symbol_persistent_only(st->symbol)) {
                    /* the persistent kernel refused this call's alignment (a
                     * caller's C or bias tensor off a 16-byte boundary) */
                    rc = pyc_hip_gemm_dispatch(general_gemm_symbol(st->dtype), st->m, st->n, st->k, vp[st->in[0]],
                                               vp[st->in[1]], out, 1.0f, beta, bias, epi, st_stream);
                }
                break;
            case ST_W8A16:
                rc = pyc_hip_w8a16_gemm_dispatch(st->symbol, st->m, st->n, st->k, vp[st->in[0]],
                                                 vp[st->in[1]], (const float*)vp[st->in[2]],
                                                 st->relu, out, st_stream);
                break;
            case ST_CONV:
                rc = pyc_hip_conv2d_dispatch(st->symbol, st->conv[0], st->conv[1], st->conv[2], st->conv[3],
                                             st->conv[4], st->conv[5], st->conv[6], st->conv[7], st->conv[8],
                                             st->conv[9], st->conv[10], vp[st->in[0]],
                                             vp[st->in[1]], bias, st->relu, out, st_stream);
                break;
            case ST_GELU:
                rc = pyc_hip_gelu_dispatch(st->symbol, st->elems, vp[st->in[0]], out, st_stream);
                break;
            case ST_LAYERNORM:
                rc = pyc_hip_layernorm_dispatch(st->symbol, st->m, st->n, st->eps, vp[st->in[0]],
                                                st->in[1] >= 0 ? vp[st->in[1]] : NULL,
                                                st->in[2] >= 0 ? vp[st->in[2]] : NULL, out, st_stream);
                break;
            case ST_ATTN: {
                const float scale = 1.0f / sqrtf((float)st->attn[3]);
                rc = pyc_hip_attention_dispatch(st->symbol, st->attn[0], st->attn[1], st->attn[2], st->attn[3],
                                                st->attn[4], vp[st->in[0]], vp[st->in[1]],
                                                vp[st->in[2]], out, scale, st_stream);
                break;
            }
            default:
                break;
        }
        if (arm) {
            *signalled = pyc_hip_run_signal_taken() && rc == 0;
        }
        if (rc != 0) {
            snprintf(why, why_cap, "hip_kernel_failed:%s", st->symbol);
            return -1;
        }
    }
    (void)m;
    return 0;
}

static int execute_native(const pyc_ir_module* m, const pyc_tensor* inputs, size_t input_count,
                          pyc_tensor* outputs, size_t output_count, pyc_cuda_dispatch_trace* trace,
                          char* why, size_t why_cap) {
    static hip_plan plan; /* guarded by g_dispatch_lock */
    const int static_lhs = env_true("PYC_CUDA_ASSUME_STATIC_LHS");
    const int static_rhs = env_true("PYC_CUDA_ASSUME_STATIC_RHS");
    const int skip_out = env_true("PYC_CUDA_SKIP_HOST_OUTPUT_COPY");
    int use_graph = env_default_true("PYC_CUDA_ENABLE_GRAPH_REPLAY");
    int copy_in[PYC_IR_MAX_OPS];
    void* vp[PYC_IR_MAX_OPS];   /* device storage of each value: workspace or the caller's device tensor */
    int dev_in[PYC_IR_MAX_OPS]; /* INPUT op bound to the caller's device tensor (no staging, no copy) */
    int dev_out[64];            /* output whose caller tensor is device memory */
    int out_d2d[64];            /* ... filled by a device-to-device copy (its value is stored elsewhere) */
    int any_dev = 0;
    int has_chain = 0;
    size_t i;
    uint64_t sig = 1469598103934665603ull, mod_sig;
    graph_slot* gs = NULL;
    int replayed = 0;
    double t0;
    float dev_ms = 0.0f;

    why[0] = '\0';
    if (build_plan(m, &plan) != 0) {
        return 1; /* unsupported pattern: not a failure of the GPU */
    }
    if (plan.n_outputs > output_count || plan.n_outputs > 64) {
        return 1;
    }
    has_chain = plan_has_chain(&plan);
    if (ws_init() != 0) {
        snprintf(why, why_cap, "hip_workspace_init_failed");
        return -1;
    }

    /* static-input uploads (uploaded[]) stay valid only while the same module
     * runs: another module's values share the per-op-id device buffers */
    mod_sig = fnv(sig, &m->op_count, sizeof(m->op_count));
    mod_sig = fnv(mod_sig, m->ops, m->op_count * sizeof(pyc_ir_op));
    if (g_ws.upload_module != mod_sig) {
        memset(g_ws.uploaded, 0, sizeof(g_ws.uploaded));
        g_ws.upload_module = mod_sig;
    }

    /* bind inputs, size checks, device + staging buffers */
    memset(vp, 0, sizeof(vp));
    memset(dev_in, 0, sizeof(dev_in));
    memset(dev_out, 0, sizeof(dev_out));
    memset(out_d2d, 0, sizeof(out_d2d));
    for (i = 0; i < m->op_count; ++i) {
        const int ord = plan.input_ordinal[i];
        size_t bytes;
        copy_in[i] = 0;
        if (ord < 0) {
            if (plan.value_bytes[i] && plan.value_op[i] == (int)i &&
                dgrow(&g_ws.val[i], plan.value_bytes[i]) != 0) {
                snprintf(why, why_cap, "hip_malloc_failed");
                return -1;
            }
            vp[i] = g_ws.val[i].ptr;
            continue;
        }
        if ((size_t)ord >= input_count || !inputs[ord].data) {
            return 1;
        }
        bytes = plan.value_bytes[i];
        if (inputs[ord].dtype != m->ops[i].dtype || inputs[ord].size_bytes < bytes) {
            return 1;
        }
        if (is_device_ptr(inputs[ord].data)) {
            dev_in[i] = 1; /* read in place */
            vp[i] = inputs[ord].data;
            continue;
        }
        if (dgrow(&g_ws.val[i], bytes) != 0 || hgrow(&g_ws.stage_in[i], bytes) != 0) {
            snprintf(why, why_cap, "hip_malloc_failed");
            return -1;
        }
        vp[i] = g_ws.val[i].ptr;
        copy_in[i] = 1;
        if (g_ws.uploaded[i] && g_ws.last_host[i] == inputs[ord].data && g_ws.last_bytes[i] == bytes &&
            ((plan.is_weight[i] && static_rhs) || (!plan.is_weight[i] && static_lhs))) {
            copy_in[i] = 0;
        }
    }
    for (i = 0; i < plan.n_outputs; ++i) {
        const int src = plan.output_src[i];
        const size_t bytes = plan.value_bytes[src];
        if (outputs[i].dtype != plan.vdtype[src]) {
            return 1; /* output dtype must match the produced value */
        }
        if (outputs[i].data && is_device_ptr(outputs[i].data)) {
            size_t j;
            int bound = plan.input_ordinal[src] >= 0; /* an input passed through: copy it */
            if (outputs[i].size_bytes < bytes) {
                return 1;
            }
            for (j = 0; j < i; ++j) {
                bound |= dev_out[j] && !out_d2d[j] && plan.output_src[j] == src; /* value already written elsewhere */
            }
            dev_out[i] = 1;
            if (bound) {
                out_d2d[i] = 1;
            } else {
                vp[src] = outputs[i].data; /* the producing step writes the caller's tensor */
            }
            continue;
        }
        if (!skip_out && (!outputs[i].data || outputs[i].size_bytes < bytes)) {
            return 1;
        }
        if (hgrow(&g_ws.stage_out[i], bytes) != 0) {
            snprintf(why, why_cap, "hip_malloc_failed");
            return -1;
        }
    }
    for (i = 0; i < m->op_count; ++i) {
        any_dev |= dev_in[i];
    }
    for (i = 0; i < plan.n_outputs; ++i) {
        any_dev |= dev_out[i];
    }
    if (any_dev) {
        /* The caller's device tensors are ordered by the default-stream
         * contract of a library call: the run starts after all work queued on
         * the legacy null stream (torch's default stream), which itself waits
         * for every blocking stream and for whatever the caller made it wait
         * for (torch: current_stream().wait_stream(side)). Work left pending
         * on other non-blocking streams is the caller's to complete first.
         * The backend's own stream is non-blocking, so this wait does not
         * touch it: hipDeviceSynchronize would, and after a run that ended on
         * the completion word HIP first retires that run with a marker round
         * trip (~8 us per call). */
        if (hipStreamSynchronize(NULL) != hipSuccess) {
            snprintf(why, why_cap, "hip_sync_failed");
            return -1;
        }
    }

    /* fp32 add operands: uploaded as part of the inputs; converted copies for half ones */
    for (i = 0; i < plan.nsteps; ++i) {
        const hip_step* st = &plan.steps[i];
        if (st->add_in >= 0 && st->add_mode != ADD_MATRIX) {
            const int ord = plan.input_ordinal[st->add_in];
            const size_t cols = st->kind == ST_CONV ? (size_t)st->conv[4] : (size_t)st->n;
            if (st->add_mode == ADD_ROW_BIAS && !plan.f32_bias_needed[st->add_in]) {
                continue; /* fp32 row bias: used in place */
            }
            if (dgrow(&g_ws.bias32[st->add_in], cols * sizeof(float)) != 0) {
                snprintf(why, why_cap, "hip_malloc_failed");
                return -1;
            }
            if (ord < 0 || (size_t)ord >= input_count) {
                return 1;
            }
            {
                /* small host-side conversion / broadcast, then one upload (an
                 * operand in device memory is first read back: it is a [N] or
                 * [1] vector) */
                float* tmp = (float*)malloc(cols * sizeof(float));
                const void* hsrc = inputs[ord].data;
                void* hcopy = NULL;
                size_t c;
                if (!tmp) {
                    return -1;
                }
                if (dev_in[st->add_in]) {
                    const size_t nb = (st->add_mode == ADD_SCALAR ? 1 : cols) * dtype_bytes(m->ops[st->add_in].dtype);
                    hcopy = malloc(nb);
                    if (!hcopy || hipMemcpy(hcopy, inputs[ord].data, nb, hipMemcpyDeviceToHost) != hipSuccess) {
                        free(hcopy);
                        free(tmp);
                        snprintf(why, why_cap, "hip_copy_failed");
                        return -1;
                    }
                    hsrc = hcopy;
                }
                for (c = 0; c < cols; ++c) {
                    const size_t src_i = st->add_mode == ADD_SCALAR ? 0 : c;
                    const pyc_dtype dt = m->ops[st->add_in].dtype;
                    if (dt == PYC_DTYPE_F32) {
                        tmp[c] = ((const float*)hsrc)[src_i];
                    } else if (dt == PYC_DTYPE_BF16) {
                        tmp[c] = bf16_bits_to_f32(((const uint16_t*)hsrc)[src_i]);
                    } else {
                        tmp[c] = f16_bits_to_f32(((const uint16_t*)hsrc)[src_i]);
                    }
                }
                free(hcopy);
                if (hipMemcpy(g_ws.bias32[st->add_in].ptr, tmp, cols * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
                    free(tmp);
                    snprintf(why, why_cap, "hip_copy_failed");
                    return -1;
                }
                free(tmp);
            }
        }
    }

    /* A plan that records one operation (one kernel step, no copies) is
     * launched directly: a graph of one node only adds launch latency. */
    if (use_graph && !has_chain) {
        size_t nodes = plan.nsteps;
        for (i = 0; i < m->op_count; ++i) {
            nodes += plan.input_ordinal[i] >= 0 && copy_in[i];
        }
        for (i = 0; i < plan.n_outputs; ++i) {
            nodes += dev_out[i] ? (size_t)out_d2d[i] : (size_t)!skip_out;
        }
        use_graph = nodes >= 2;
    }

    /* run signature: module content + device pointers + copy flags */
    sig = mod_sig;
    sig = fnv(sig, &skip_out, sizeof(skip_out));
    sig = fnv(sig, &g_tune_gen, sizeof(g_tune_gen));
    /* the planned kernels: an env or registry change of a symbol recaptures */
    for (i = 0; i < plan.nsteps; ++i) {
        sig = fnv(sig, plan.steps[i].symbol, strlen(plan.steps[i].symbol));
        sig = fnv(sig, &plan.steps[i].chain_len, sizeof(int));
    }
    for (i = 0; i < m->op_count; ++i) {
        if (plan.input_ordinal[i] >= 0) {
            sig = fnv(sig, &copy_in[i], sizeof(int));
            sig = fnv(sig, &dev_in[i], sizeof(int));
        }
    }
    /* a graph bakes in the caller's device tensors: their addresses are part of the run */
    sig = fnv(sig, vp, m->op_count * sizeof(vp[0]));
    for (i = 0; i < plan.n_outputs; ++i) {
        sig = fnv(sig, &dev_out[i], sizeof(int));
        if (dev_out[i]) {
            sig = fnv(sig, &outputs[i].data, sizeof(void*));
        }
    }

    /* kernel_ms: by default the host time of the enqueue, as the reference
     * measures it (cuda_backend.c:1822-1825); PYC_HIP_KERNEL_EVENTS=1 records
     * HIP events around the work instead and reports device time. Two event
     * records cost ~4.4 us per run on MI355X, a third of a small GEMM's call. */
    const int use_ev = trace && env_true("PYC_HIP_KERNEL_EVENTS");
    double t_enq = 0.0;
    /* completion word: see the wait below */
    int signal = !use_ev && !has_chain;
    int signalled = 0;
    uint32_t done_seq = 0;
    for (i = 0; signal && i < plan.n_outputs; ++i) {
        signal = dev_out[i] || skip_out;
    }
    if (signal) {
        done_seq = ++g_ws.done_seq == 0 ? ++g_ws.done_seq : g_ws.done_seq; /* 0 is the initial word */
    }

    /* host -> pinned staging */
    t0 = now_ms();
    for (i = 0; i < m->op_count; ++i) {
        const int ord = plan.input_ordinal[i];
        if (ord >= 0 && copy_in[i]) {
            memcpy(g_ws.stage_in[i].ptr, inputs[ord].data, plan.value_bytes[i]);
        }
    }
    if (trace) {
        trace->copy_in_ms += now_ms() - t0;
    }

    gs = use_graph ? graph_find(sig) : NULL;
    if (gs) {
        replayed = 1;
    } else {
        /* record: either into a new graph or directly */
        hipError_t cerr = hipSuccess;
        if (use_graph) {
            /* the fp8 GEMM's split-K workspace cannot be allocated inside a capture */
            for (i = 0; i < plan.nsteps; ++i) {
                const size_t clen = (size_t)plan.steps[i].chain_len;
                if (clen >= 2) {
                    int cn[HIP_CHAIN_MAX_STEPS], ck[HIP_CHAIN_MAX_STEPS];
                    size_t c;
                    for (c = 0; c < clen; ++c) {
                        cn[c] = plan.steps[i + c].n;
                        ck[c] = plan.steps[i + c].k;
                    }
                    (void)pyc_hip_w8a16_chain_reserve(plan.steps[i].m, (int)clen, cn, ck);
                    i += clen - 1;
                } else if (plan.steps[i].kind == ST_W8A16) {
                    (void)pyc_hip_w8a16_reserve(plan.steps[i].n, plan.steps[i].k);
                }
            }
            cerr = hipStreamBeginCapture(g_ws.stream, hipStreamCaptureModeThreadLocal);
        }
        if (cerr == hipSuccess) {
            int rc = 0;
            for (i = 0; i < m->op_count && rc == 0; ++i) {
                if (plan.input_ordinal[i] >= 0 && copy_in[i]) {
                    if (hipMemcpyAsync(g_ws.val[i].ptr, g_ws.stage_in[i].ptr, plan.value_bytes[i],
                                       hipMemcpyHostToDevice, g_ws.stream) != hipSuccess) {
                        rc = -1;
                    }
                }
            }
            if (rc == 0 && !use_graph && use_ev) {
                rc = hipEventRecord(g_ws.ev0, g_ws.stream) == hipSuccess ? 0 : -1;
            }
            if (rc == 0) {
                const double te = now_ms();
                /* the kernel may carry the completion word when nothing
                 * follows it on the stream */
                int arm = signal && !use_graph;
                for (i = 0; arm && i < plan.n_outputs; ++i) {
                    arm = !(dev_out[i] && out_d2d[i]);
                }
                rc = enqueue_steps(m, &plan, vp, arm ? done_seq : 0u, &signalled, why, why_cap);
                if (!use_graph) {
                    t_enq += now_ms() - te;
                }
            }
            if (rc == 0 && !use_graph && use_ev) {
                rc = hipEventRecord(g_ws.ev1, g_ws.stream) == hipSuccess ? 0 : -1;
            }
            if (rc == 0 && has_chain && pyc_hip_w8a16_chain_error_enqueue(g_ws.chain_err, g_ws.stream) != 0) {
                rc = -1; /* the chain's timeout word is read back with every run */
            }
            for (i = 0; rc == 0 && i < plan.n_outputs; ++i) {
                const int src = plan.output_src[i];
                if (dev_out[i]) {
                    if (out_d2d[i] && hipMemcpyAsync(outputs[i].data, vp[src], plan.value_bytes[src],
                                                     hipMemcpyDeviceToDevice, g_ws.stream) != hipSuccess) {
                        rc = -1;
                    }
                } else if (!skip_out && hipMemcpyAsync(g_ws.stage_out[i].ptr, vp[src], plan.value_bytes[src],
                                                       hipMemcpyDeviceToHost, g_ws.stream) != hipSuccess) {
                    rc = -1;
                }
            }
            if (use_graph) {
                hipGraph_t graph = NULL;
                hipGraphExec_t exec = NULL;
                hipError_t e = hipStreamEndCapture(g_ws.stream, &graph);
                if (rc == 0 && e == hipSuccess && graph &&
                    hipGraphInstantiate(&exec, graph, NULL, NULL, 0) == hipSuccess) {
                    gs = graph_victim();
                    gs->graph = graph;
                    gs->exec = exec;
                    gs->sig = sig;
                    gs->last_use = ++g_ws.graph_clock;
                    gs->valid = 1;
                } else {
                    if (graph) {
                        (void)hipGraphDestroy(graph);
                    }
                    if (why[0] == '\0') {
                        snprintf(why, why_cap, "hip_graph_capture_failed");
                    }
                    return -1;
                }
            } else if (rc != 0) {
                if (why[0] == '\0') {
                    snprintf(why, why_cap, "hip_enqueue_failed");
                }
                return -1;
            }
        } else {
            snprintf(why, why_cap, "hip_graph_begin_failed");
            return -1;
        }
    }

    t0 = now_ms();
    if (use_graph) {
        if ((use_ev && hipEventRecord(g_ws.ev0, g_ws.stream) != hipSuccess) ||
            hipGraphLaunch(gs->exec, g_ws.stream) != hipSuccess ||
            (use_ev && hipEventRecord(g_ws.ev1, g_ws.stream) != hipSuccess)) {
            snprintf(why, why_cap, "hip_graph_launch_failed");
            return -1;
        }
        t_enq += now_ms() - t0;
    }
    /* The wait. A run whose results all stay in device memory (no copy into
     * host staging, no chain timeout word to read back, no timing events)
     * waits on a completion word stored behind its work: by its last kernel
     * itself where that kernel can (signalled), else by run_signal.hip's
     * one-lane kernel; either is ~4.6 us sooner after the work than
     * hipStreamSynchronize on this stack. The others synchronize the stream. */
    {
        if (signal) {
            if ((!signalled && pyc_hip_run_signal_enqueue(g_ws.done_word, done_seq, g_ws.stream) != 0) ||
                wait_done_word(done_seq) != 0) {
                snprintf(why, why_cap, "hip_sync_failed");
                return -1;
            }
        } else if (hipStreamSynchronize(g_ws.stream) != hipSuccess) {
            snprintf(why, why_cap, "hip_sync_failed");
            return -1;
        }
    }
    if (has_chain && *g_ws.chain_err != 0) {
        /* A chain workgroup gave up waiting for another one (the grid was not
         * all resident): the outputs are invalid. Clear the word and fail the
         * run, so the native-failure contract applies (workspace release, CPU
         * fallback, or an error for device tensors / strict mode). */
        *g_ws.chain_err = 0;
        (void)pyc_hip_w8a16_chain_error(1);
        snprintf(why, why_cap, "hip_chain_wait_timeout");
        return -1;
    }
    if (trace) {
        trace->sync_ms += now_ms() - t0;
        if (!use_ev) {
            trace->kernel_ms += t_enq;
        } else if (hipEventElapsedTime(&dev_ms, g_ws.ev0, g_ws.ev1) == hipSuccess) {
            trace->kernel_ms += (double)dev_ms;
        }
        trace->graph_replayed = replayed;
    }

    /* pinned staging -> caller buffers */
    t0 = now_ms();
    for (i = 0; !skip_out && i < plan.n_outputs; ++i) {
        if (!dev_out[i]) {
            memcpy(outputs[i].data, g_ws.stage_out[i].ptr, plan.value_bytes[plan.output_src[i]]);
        }
    }
    if (trace) {
        trace->copy_out_ms += now_ms() - t0;
    }
    for (i = 0; i < m->op_count; ++i) {
        const int ord = plan.input_ordinal[i];
        if (ord >= 0 && copy_in[i]) {
            g_ws.uploaded[i] = 1;
            g_ws.last_host[i] = inputs[ord].data;
            g_ws.last_bytes[i] = plan.value_bytes[i];
        }
    }

    {
        const char* base = replayed ? "hip_native_graph_replay" : (use_graph ? "hip_native_graph_capture" : "hip_native");
        const char* sym = NULL;
        for (i = 0; i < plan.nsteps; ++i) {
            if (plan.steps[i].kind == ST_GEMM || plan.steps[i].kind == ST_W8A16) {
                sym = plan.steps[i].chain_len >= 2 ? "hip_w8a16_chain_e4m3" : plan.steps[i].symbol;
                break;
            }
        }
        if (!sym && plan.nsteps > 0) {
            sym = plan.steps[0].symbol;
        }
        if (sym) {
            snprintf(why, why_cap, "%s:%s", base, sym);
        } else {
            set_reason(why, why_cap, base);
        }
    }
    return 0;
}

/* ---------------------------------------------------------------- simulated executor */

/* PYC_CUDA_SIMULATE_AVAILABLE: a host-only stand-in for the GPU that lets the
 * dispatch contract be exercised without a device (reference
 * cuda_backend.c:1413-1671): naive fp32 matmul, broadcast add, relu, and
 * byte-exact passthrough of any dtype. It never runs unless that variable is
 * set, and its runs are reported as "cuda_native_simulated". */
static int execute_simulated(const pyc_ir_module* m, const pyc_tensor* inputs, size_t input_count,
                             pyc_tensor* outputs, size_t output_count) {
    const void* val[PYC_IR_MAX_OPS];
    void* owned[PYC_IR_MAX_OPS];
    size_t bytes[PYC_IR_MAX_OPS];
    size_t i, nin = 0, nout = 0;
    int fail = 0;
    memset(owned, 0, sizeof(owned));
    memset(val, 0, sizeof(val));
    for (i = 0; i < m->op_count && !fail; ++i) {
        const pyc_ir_op* op = &m->ops[i];
        const size_t elems = shape_elems(&op->shape);
        switch (op->kind) {
            case PYC_IR_OP_INPUT:
                if (nin >= input_count || !inputs[nin].data || inputs[nin].dtype != op->dtype ||
                    inputs[nin].size_bytes < elems * dtype_bytes(op->dtype) || elems == 0) {
                    fail = 1;
                    break;
                }
                val[i] = inputs[nin].data;
                bytes[i] = elems * dtype_bytes(op->dtype);
                nin++;
                break;
            case PYC_IR_OP_MATMUL: {
                const int a = op->input_ids[0], b = op->input_ids[1];
                size_t M, K, N, r, c, t;
                float* out;
                if (op->input_count < 2 || !valid_id(m, a) || !valid_id(m, b) || !val[a] || !val[b] ||
                    op->dtype != PYC_DTYPE_F32 || m->ops[a].shape.rank != 2 || m->ops[b].shape.rank != 2 ||
                    m->ops[a].shape.dims[1] != m->ops[b].shape.dims[0]) {
                    fail = 1;
                    break;
                }
                M = (size_t)m->ops[a].shape.dims[0];
                K = (size_t)m->ops[a].shape.dims[1];
                N = (size_t)m->ops[b].shape.dims[1];
                out = (float*)malloc(M * N * sizeof(float));
                if (!out) {
                    fail = 1;
                    break;
                }
                for (r = 0; r < M; ++r) {
                    for (c = 0; c < N; ++c) {
                        float acc = 0.0f;
                        for (t = 0; t < K; ++t) {
                            acc += ((const float*)val[a])[r * K + t] * ((const float*)val[b])[t * N + c];
                        }
                        out[r * N + c] = acc;
                    }
                }
                owned[i] = out;
                val[i] = out;
                bytes[i] = M * N * sizeof(float);
                break;
            }
            case PYC_IR_OP_ADD: {
                const int a = op->input_ids[0], b = op->input_ids[1];
                size_t na, nb, j;
                float* out;
                if (op->input_count < 2 || !valid_id(m, a) || !valid_id(m, b) || !val[a] || !val[b] ||
                    op->dtype != PYC_DTYPE_F32) {
                    fail = 1;
                    break;
                }
                na = bytes[a] / sizeof(float);
                nb = bytes[b] / sizeof(float);
                if (nb > na) {
                    const int tmp = a;
                    (void)tmp;
                    fail = 1;
                    break;
                }
                out = (float*)malloc(na * sizeof(float));
                if (!out || nb == 0 || na % nb != 0) {
                    free(out);
                    fail = 1;
                    break;
                }
                for (j = 0; j < na; ++j) {
                    out[j] = ((const float*)val[a])[j] + ((const float*)val[b])[j % nb];
                }
                owned[i] = out;
                val[i] = out;
                bytes[i] = na * sizeof(float);
                break;
            }
            case PYC_IR_OP_RELU: {
                const int a = op->input_ids[0];
                size_t n, j;
                float* out;
                if (op->input_count < 1 || !valid_id(m, a) || !val[a] || op->dtype != PYC_DTYPE_F32) {
                    fail = 1;
                    break;
                }
                n = bytes[a] / sizeof(float);
                out = (float*)malloc(n * sizeof(float));
                if (!out) {
                    fail = 1;
                    break;
                }
                for (j = 0; j < n; ++j) {
                    const float v = ((const float*)val[a])[j];
                    out[j] = v > 0.0f ? v : 0.0f;
                }
                owned[i] = out;
                val[i] = out;
                bytes[i] = n * sizeof(float);
                break;
            }
            case PYC_IR_OP_OUTPUT: {
                const int a = op->input_ids[0];
                if (op->input_count < 1 || !valid_id(m, a) || !val[a] || nout >= output_count ||
                    !outputs[nout].data || outputs[nout].size_bytes < bytes[a]) {
                    fail = 1;
                    break;
                }
                memcpy(outputs[nout].data, val[a], bytes[a]);
                nout++;
                break;
            }
            default:
                fail = 1;
                break;
        }
    }
    for (i = 0; i < m->op_count; ++i) {
        free(owned[i]);
    }
    return fail ? -1 : 0;
}

/* ---------------------------------------------------------------- dispatch */

static int native_kind_supported(const pyc_ir_module* m) {
    size_t i;
    if (!m || m->op_count == 0) {
        return 0;
    }
    for (i = 0; i < m->op_count; ++i) {
        switch (m->ops[i].kind) {
            case PYC_IR_OP_INPUT:
            case PYC_IR_OP_MATMUL:
            case PYC_IR_OP_ADD:
            case PYC_IR_OP_RELU:
            case PYC_IR_OP_OUTPUT:
            case PYC_IR_OP_CONV2D:
            case PYC_IR_OP_ATTENTION:
            case PYC_IR_OP_GELU:
            case PYC_IR_OP_LAYERNORM:
                break;
            default:
                return 0;
        }
        if (dtype_bytes(m->ops[i].dtype) == 0 && m->ops[i].kind != PYC_IR_OP_OUTPUT) {
            return 0;
        }
    }
    return 1;
}

static pyc_cuda_dispatch_status dispatch_locked(const pyc_ir_module* module, const pyc_tensor* inputs,
                                                size_t input_count, pyc_tensor* outputs, size_t output_count,
                                                pyc_cpu_executor_fn cpu_executor, void* executor_ctx,
                                                pyc_cuda_dispatch_trace* trace) {
    char reason[PYC_CUDA_REASON_MAX];
    char native[PYC_CUDA_REASON_MAX];
    int available;
    int supported;
    int native_rc = 1;
    int dev_tensors = 0;

    if (!module || !inputs || !outputs || !cpu_executor) {
        return PYC_CUDA_DISPATCH_ERROR;
    }
    pyc_cuda_dispatch_trace_init(trace);
    if (trace) {
        trace->cuda_requested = 1;
    }
    if (env_true("PYC_CUDA_FORCE_ERROR")) {
        if (trace) {
            trace->cuda_available = 0;
            trace->fallback_to_cpu = 0;
            set_reason(trace->reason, sizeof(trace->reason), "forced_error");
        }
        return PYC_CUDA_DISPATCH_ERROR;
    }
    reason[0] = '\0';
    native[0] = '\0';
    available = detect_gpu(reason, sizeof(reason));
    if (trace) {
        trace->cuda_available = available;
    }
    supported = native_kind_supported(module);
    /* Tensors in device memory (an extension: the reference takes host
     * pointers only) can be run only natively; the simulated and CPU
     * executors read host memory. */
    dev_tensors = available && any_device_tensor(inputs, input_count, outputs, output_count);
    if (available && supported && !env_true("PYC_CUDA_FORCE_FALLBACK")) {
        int count = 0;
        /* a real device is tried first, also when the simulation flag is set
         * (reference cuda_backend.c:2856-2880) */
        if (device_count(&count) == 0 && count > 0) {
            native_rc = execute_native(module, inputs, input_count, outputs, output_count, trace, native,
                                       sizeof(native));
            if (native_rc == 0) {
                if (trace) {
                    trace->fallback_to_cpu = 0;
                    set_reason(trace->reason, sizeof(trace->reason), native);
                }
                return PYC_CUDA_DISPATCH_OK;
            }
            if (native_rc < 0) {
                ws_release();
            }
        }
        if (!dev_tensors && env_true("PYC_CUDA_SIMULATE_AVAILABLE") &&
            execute_simulated(module, inputs, input_count, outputs, output_count) == 0) {
            if (trace) {
                trace->fallback_to_cpu = 0;
                set_reason(trace->reason, sizeof(trace->reason), "cuda_native_simulated");
            }
            return PYC_CUDA_DISPATCH_OK;
        }
    }

    if (dev_tensors) {
        if (trace) {
            trace->fallback_to_cpu = 0;
            if (native[0] != '\0') {
                snprintf(trace->reason, sizeof(trace->reason), "%.90s;device_tensors_no_cpu_fallback", native);
            } else {
                set_reason(trace->reason, sizeof(trace->reason), "device_tensors_no_cpu_fallback");
            }
        }
        return PYC_CUDA_DISPATCH_ERROR;
    }
    if (cpu_executor(module, inputs, input_count, outputs, output_count, executor_ctx) != 0) {
        if (trace) {
            trace->fallback_to_cpu = 0;
            if (native[0] != '\0') {
                snprintf(trace->reason, sizeof(trace->reason), "%.100s;cpu_fallback_failed", native);
            } else {
                set_reason(trace->reason, sizeof(trace->reason), "cpu_fallback_failed");
            }
        }
        return PYC_CUDA_DISPATCH_ERROR;
    }
    if (trace) {
        trace->fallback_to_cpu = 1;
        if (env_true("PYC_CUDA_FORCE_FALLBACK")) {
            set_reason(trace->reason, sizeof(trace->reason), "cuda_forced_fallback");
        } else if (available && (!supported || native_rc > 0)) {
            set_reason(trace->reason, sizeof(trace->reason), "cuda_native_unsupported_fallback");
        } else if (available) {
            set_reason(trace->reason, sizeof(trace->reason), "cuda_native_failed_fallback");
        } else {
            set_reason(trace->reason, sizeof(trace->reason), reason);
        }
    }
    return PYC_CUDA_DISPATCH_FALLBACK;
}

pyc_cuda_dispatch_status pyc_cuda_dispatch(const pyc_ir_module* module, const pyc_tensor* inputs,
                                           size_t input_count, pyc_tensor* outputs, size_t output_count,
                                           pyc_cpu_executor_fn cpu_executor, void* executor_ctx,
                                           pyc_cuda_dispatch_trace* trace) {
    pyc_cuda_dispatch_status st;
    pyc_mutex_lock(&g_dispatch_lock);
    st = dispatch_locked(module, inputs, input_count, outputs, output_count, cpu_executor, executor_ctx, trace);
    pyc_mutex_unlock(&g_dispatch_lock);
    return st;
}

/* Releases every device/pinned buffer, the stream and the captured graph. */
/* Measured autotune of the [M,K]x[K,N] GEMM (reference compiler_api.c:3000-3044
 * records an estimate per run instead): every registered variant of the dtype
 * with a [K,N] right operand is launched `iters` times at the live shape on
 * scratch operands, timed by HIP events, and the fastest becomes the plan's
 * symbol for that shape. Returns the number of timed variants (symbols and
 * mean ms in syms/ms), 0 when nothing could be timed, -1 on bad arguments. */
/* Fills `bytes` of device memory with uniform values in [-1, 1) of `dtype`
 * (xorshift64; [0, 1) with nonneg, as activations after a ReLU), a 1 MiB
 * host pattern repeated: timing on real-looking data,
 * since constant operands switch less logic, draw less power and let the
 * clock run higher than a model's data does. */
static int fill_operand(void* dst, size_t bytes, pyc_dtype dtype, uint64_t seed, int nonneg) {
    const size_t chunk = (size_t)1 << 20;
    uint8_t* pat = (uint8_t*)malloc(chunk);
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    size_t i, off;
    int rc = 0;
    if (!pat) {
        return -1;
    }
    for (i = 0; i < chunk / 4; ++i) {
        float f;
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        f = (float)((double)(x >> 40) / (double)(1ull << 24));
        if (!nonneg) {
            f = f * 2.0f - 1.0f;
        }
        if (dtype == PYC_DTYPE_F32) {
            memcpy(pat + 4 * i, &f, 4);
        } else {
            uint16_t h[2];
            uint32_t u;
            memcpy(&u, &f, 4);
            if (dtype == PYC_DTYPE_BF16) {
                h[0] = (uint16_t)(u >> 16);
                h[1] = (uint16_t)((u >> 16) ^ 0x0080u); /* exponent bit flipped: a second value */
            } else {
                /* |f| < 1: fp16 bits from the fp32 exponent and top mantissa */
                const int e = (int)((u >> 23) & 0xff) - 127 + 15;
                const uint16_t sgn = (uint16_t)((u >> 16) & 0x8000u);
                h[0] = e <= 0 ? sgn : (uint16_t)(sgn | (uint16_t)(e << 10) | (uint16_t)((u >> 13) & 0x3ffu));
                h[1] = (uint16_t)(h[0] ^ 0x0100u);
            }
            memcpy(pat + 4 * i, h, 4);
        }
    }
    for (off = 0; off < bytes && rc == 0; off += chunk) {
        const size_t n = bytes - off < chunk ? bytes - off : chunk;
        rc = hipMemcpy((uint8_t*)dst + off, pat, n, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
    }
    free(pat);
    return rc;
}

static int cmp_double(const void* a, const void* b) {
    const double x = *(const double*)a, y = *(const double*)b;
    return x < y ? -1 : x > y;
}

/* Times candidate launches for the autotune entry points: each live
 * candidate once (which also loads its code), a settle phase on the first live
 * one (the clock of an idle card ramps over the first tens of milliseconds of
 * load: 50 ms, at most 2000 launches), then ROUNDS interleaved rounds of
 * `iters` launches per candidate, each candidate's time its median round, so
 * a clock or power drift during tuning spreads over all candidates instead of
 * favouring one. launch(i) enqueues candidate i on s and returns 0. On return
 * live[i] says whether candidate i was timed and ms[i] is its median ms. */
#define TUNE_ROUNDS 3
static void time_candidates(int ncand, int (*launch)(int i, void* ctx, hipStream_t s), void* ctx, hipStream_t s,
                            hipEvent_t e0, hipEvent_t e1, int iters, int* live, double* ms) {
    double t_round[32][TUNE_ROUNDS];
    int i, r, first = -1;
    for (i = 0; i < ncand && i < 32; ++i) {
        live[i] = live[i] && launch(i, ctx, s) == 0;
        if (live[i] && first < 0) {
            first = i;
        }
    }
    if (first >= 0) {
        const double t_end = now_ms() + 50.0;
        int launches = 0;
        while (now_ms() < t_end && launches < 2000) {
            int j;
            for (j = 0; j < 4; ++j, ++launches) {
                (void)launch(first, ctx, s);
            }
            (void)hipStreamSynchronize(s);
        }
    }
    for (r = 0; r < TUNE_ROUNDS; ++r) {
        for (i = 0; i < ncand && i < 32; ++i) {
            float t = 0.0f;
            int it, ok;
            if (!live[i]) {
                continue;
            }
            ok = hipEventRecord(e0, s) == hipSuccess;
            for (it = 0; ok && it < iters; ++it) {
                ok = launch(i, ctx, s) == 0;
            }
            ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
                 hipEventElapsedTime(&t, e0, e1) == hipSuccess;
            if (!ok) {
                live[i] = 0;
                continue;
            }
            t_round[i][r] = (double)t / iters;
        }
    }
    for (i = 0; i < ncand && i < 32; ++i) {
        if (live[i]) {
            qsort(t_round[i], TUNE_ROUNDS, sizeof(double), cmp_double);
            ms[i] = t_round[i][TUNE_ROUNDS / 2];
        }
    }
}

/* Records (key -> best) in a tuned table, replacing the key's entry or, when
 * the table is full, its last slot. */
static void tuned_store(tuned_entry* tab, int* count, int cap, const tuned_entry* e) {
    int slot = *count, j;
    for (j = 0; j < *count; ++j) {
        if (memcmp(tab[j].key, e->key, sizeof(e->key)) == 0) {
            slot = j;
        }
    }
    if (slot == cap) {
        slot = cap - 1;
    } else if (slot == *count) {
        (*count)++;
    }
    tab[slot] = *e;
    g_tune_gen++;
}

typedef struct {
    const char* const* cands;
    int M, N, K;
    void *a, *b, *c;
} gemm_tune_ctx;

static int gemm_tune_launch(int i, void* ctx, hipStream_t s) {
    const gemm_tune_ctx* g = (const gemm_tune_ctx*)ctx;
    return pyc_hip_gemm_dispatch(g->cands[i], g->M, g->N, g->K, g->a, g->b, g->c, 1.0f, 0.0f, NULL, 0, s);
}

/* Writes the timed candidates (symbol, median ms) to syms/ms and returns the
 * index of the fastest in cands, or -1. */
static int tune_report(const char* const* cands, int ncand, const int* live, const double* t, char* syms,
                       size_t sym_stride, double* ms, int cap, int* n) {
    int i, best = -1;
    *n = 0;
    for (i = 0; i < ncand && *n < cap; ++i) {
        if (!live[i]) {
            continue;
        }
        set_reason(syms + (size_t)(*n) * sym_stride, sym_stride, cands[i]);
        ms[*n] = t[i];
        if (best < 0 || t[i] < t[best]) {
            best = i;
        }
        ++(*n);
    }
    return best;
}

int pyc_hip_autotune_gemm(pyc_dtype dtype, int M, int N, int K, int iters, char* syms, size_t sym_stride,
                          double* ms, int cap) {
    /* one entry per distinct kernel: the reference's fp32 alias
     * ada_gemm_k64_warp32_async_f32 runs hip_gemm_f32_nn_64x64's kernel with a
     * narrower epilogue, so timing it would only pick between equal launches */
    static const char* const cands[] = {"hip_gemm_bf16_nn_256x256_lds", "hip_gemm_bf16_nn_256x256",
                                        "hip_gemm_bf16_nn_128x128", "hip_gemm_bf16_nn", "cutlass_gemm_tensorcore_bf16",
                                        "hip_gemm_f16_nn_256x256_lds", "hip_gemm_f16_nn", "hip_gemm_f32_nn_64x64"};
    enum { NCAND = sizeof(cands) / sizeof(cands[0]) };
    const size_t eb = dtype_bytes(dtype);
    gemm_tune_ctx g;
    hipStream_t s = NULL;
    hipEvent_t e0 = NULL, e1 = NULL;
    int devices = 0;
    double t[NCAND];
    int live[NCAND];
    int n = 0, best;
    size_t i;
    if ((dtype != PYC_DTYPE_F32 && dtype != PYC_DTYPE_BF16 && dtype != PYC_DTYPE_F16) || M <= 0 || N <= 0 ||
        K <= 0 || iters <= 0 || !syms || sym_stride == 0 || !ms || cap <= 0) {
        return -1;
    }
    if (env_true("PYC_CUDA_DISABLE") || hipGetDeviceCount(&devices) != hipSuccess || devices <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    memset(&g, 0, sizeof(g));
    g.cands = cands;
    g.M = M;
    g.N = N;
    g.K = K;
    pyc_mutex_lock(&g_dispatch_lock);
    if (hipMalloc(&g.a, (size_t)M * K * eb) != hipSuccess || hipMalloc(&g.b, (size_t)K * N * eb) != hipSuccess ||
        hipMalloc(&g.c, (size_t)M * N * eb) != hipSuccess || hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess ||
        fill_operand(g.a, (size_t)M * K * eb, dtype, 1, 0) != 0 || fill_operand(g.b, (size_t)K * N * eb, dtype, 2, 0) != 0) {
        goto done;
    }
    /* candidates of this dtype (whether the shape meets their preconditions
     * shows in their first launch) */
    for (i = 0; i < NCAND; ++i) {
        live[i] = dtype == PYC_DTYPE_BF16 ? strstr(cands[i], "bf16") != NULL
                  : dtype == PYC_DTYPE_F16 ? strstr(cands[i], "f16") != NULL && !strstr(cands[i], "bf16")
                                           : strstr(cands[i], "f32") != NULL;
    }
    time_candidates(NCAND, gemm_tune_launch, &g, s, e0, e1, iters, live, t);
    best = tune_report(cands, NCAND, live, t, syms, sym_stride, ms, cap, &n);
    if (best >= 0) {
        tuned_entry e;
        memset(&e, 0, sizeof(e));
        e.key[0] = (int)dtype;
        e.key[1] = M;
        e.key[2] = N;
        e.key[3] = K;
        set_reason(e.symbol, sizeof(e.symbol), cands[best]);
        tuned_store(g_tuned, &g_tuned_count, TUNED_MAX, &e);
    }
done:
    if (s) {
        (void)hipStreamSynchronize(s);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (g.a) (void)hipFree(g.a);
    if (g.b) (void)hipFree(g.b);
    if (g.c) (void)hipFree(g.c);
    (void)hipGetLastError();
    pyc_mutex_unlock(&g_dispatch_lock);
    return n;
}

typedef struct {
    const char* const* cands;
    int cv[11]; /* N H W C K R S ph pw sh sw */
    void *x, *w, *y;
    float* bias;
} conv_tune_ctx;

static int conv_tune_launch(int i, void* ctx, hipStream_t s) {
    const conv_tune_ctx* g = (const conv_tune_ctx*)ctx;
    const int* c = g->cv;
    return pyc_hip_conv2d_dispatch(g->cands[i], c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], c[8], c[9], c[10],
                                   g->x, g->w, g->bias, 1, g->y, s);
}

int pyc_hip_autotune_conv2d(pyc_dtype dtype, int N, int H, int W, int C_in, int K, int R, int S, int pad_h,
                            int pad_w, int stride_h, int stride_w, int iters, char* syms, size_t sym_stride,
                            double* ms, int cap) {
    /* the distinct paths (the reference's names are aliases of the first) */
    static const char* const cands[] = {"hip_conv2d_bf16", "hip_conv2d_bf16_persist", "hip_conv2d_bf16_tiled",
                                        "hip_conv2d_f16", "hip_conv2d_f16_persist", "hip_conv2d_f16_tiled"};
    enum { NCAND = sizeof(cands) / sizeof(cands[0]) };
    conv_tune_ctx g;
    hipStream_t s = NULL;
    hipEvent_t e0 = NULL, e1 = NULL;
    int devices = 0;
    double t[NCAND];
    int live[NCAND];
    int n = 0, best;
    size_t i, xb, wb, yb;
    int64_t P, Q;
    if ((dtype != PYC_DTYPE_BF16 && dtype != PYC_DTYPE_F16) || N <= 0 || H <= 0 || W <= 0 || C_in <= 0 || K <= 0 ||
        R <= 0 || S <= 0 || pad_h < 0 || pad_w < 0 || stride_h <= 0 || stride_w <= 0 || H + 2 * pad_h < R ||
        W + 2 * pad_w < S || iters <= 0 || !syms || sym_stride == 0 || !ms || cap <= 0) {
        return -1;
    }
    if (env_true("PYC_CUDA_DISABLE") || hipGetDeviceCount(&devices) != hipSuccess || devices <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    P = (H + 2 * pad_h - R) / stride_h + 1;
    Q = (W + 2 * pad_w - S) / stride_w + 1;
    xb = (size_t)N * H * W * C_in * 2;
    wb = (size_t)K * R * S * C_in * 2;
    yb = (size_t)N * (size_t)P * (size_t)Q * K * 2;
    memset(&g, 0, sizeof(g));
    g.cands = cands;
    g.cv[0] = N; g.cv[1] = H; g.cv[2] = W; g.cv[3] = C_in; g.cv[4] = K; g.cv[5] = R; g.cv[6] = S;
    g.cv[7] = pad_h; g.cv[8] = pad_w; g.cv[9] = stride_h; g.cv[10] = stride_w;
    pyc_mutex_lock(&g_dispatch_lock);
    if (hipMalloc(&g.x, xb) != hipSuccess || hipMalloc(&g.w, wb) != hipSuccess || hipMalloc(&g.y, yb) != hipSuccess ||
        hipMalloc((void**)&g.bias, (size_t)K * sizeof(float)) != hipSuccess ||
        hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
        hipEventCreate(&e1) != hipSuccess || fill_operand(g.x, xb, dtype, 1, 1) != 0 ||
        fill_operand(g.w, wb, dtype, 2, 0) != 0 || fill_operand(g.bias, (size_t)K * sizeof(float), PYC_DTYPE_F32, 3, 0) != 0) {
        goto done;
    }
    for (i = 0; i < NCAND; ++i) {
        live[i] = (strstr(cands[i], "bf16") != NULL) == (dtype == PYC_DTYPE_BF16);
    }
    time_candidates(NCAND, conv_tune_launch, &g, s, e0, e1, iters, live, t);
    best = tune_report(cands, NCAND, live, t, syms, sym_stride, ms, cap, &n);
    if (best >= 0) {
        tuned_entry e;
        memset(&e, 0, sizeof(e));
        e.key[0] = (int)dtype;
        memcpy(&e.key[1], g.cv, sizeof(g.cv));
        set_reason(e.symbol, sizeof(e.symbol), cands[best]);
        tuned_store(g_tuned_conv, &g_tuned_conv_count, TUNED_MAX, &e);
    }
done:
    if (s) {
        (void)hipStreamSynchronize(s);
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (g.x) (void)hipFree(g.x);
    if (g.w) (void)hipFree(g.w);
    if (g.y) (void)hipFree(g.y);
    if (g.bias) (void)hipFree(g.bias);
    (void)hipGetLastError();
    pyc_mutex_unlock(&g_dispatch_lock);
    return n;
}

void pyc_hip_backend_release(void) {
    pyc_mutex_lock(&g_dispatch_lock);
    ws_release();
    pyc_mutex_unlock(&g_dispatch_lock);
}
