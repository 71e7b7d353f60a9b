/* kernel_registry.c — process-wide kernel candidate table.
 *
 * Behaviour follows reference src/compiler/runtime/kernel_registry.c:
 *   - 512 slots, first free slot on register, descriptors copied by value (:204-222);
 *   - score = 100*priority + occupancy*(12 in UTILIZATION_FIRST else 6)
 *             + 25 if MFMA/tensor-core eligible - 100*best_ms (once measured)
 *             - pressure*(LDS KiB + 8*reg class)  (not in UTILIZATION_FIRST)  (:161-172);
 *   - joint score additionally subtracts the allocator penalty, adds the reuse
 *     bonus and the workload (+36/-18) and hardware (+48/-8/+10/-24) affinity
 *     terms (:54-199);
 *   - ties go to the lexically smaller symbol; collect returns symbols in
 *     lexical order (:318-454, :518-561);
 *   - promotion marks exactly one symbol per (op, backend) (:224-268).
 * The coefficients are kept identical because the selections they produce are
 * part of the reference's tested contract (tests/compiler_next/test_kernel_registry.c).
 * Differences: the table is guarded by a mutex (the reference's is not), and
 * PYC_KERNEL_HARDWARE_CDNA4 is named "cdna4". */
#include "pyc/kernel_registry.h"

#include <float.h>
#include <string.h>

#include "pyc_mutex.h"

typedef struct {
    int used;
    int promoted;
    pyc_kernel_desc desc;
    pyc_kernel_benchmark bench;
} reg_entry;

static reg_entry g_table[PYC_KERNEL_MAX];
static pyc_mutex g_table_lock = PYC_MUTEX_INIT;

const char* pyc_kernel_workload_family_name(pyc_kernel_workload_family family) {
    static const char* const names[] = {"any", "small", "square", "large_square", "tall_skinny", "wide_skinny"};
    if ((int)family < 0 || (int)family > (int)PYC_KERNEL_WORKLOAD_WIDE_SKINNY) {
        return "any";
    }
    return names[family];
}

const char* pyc_kernel_hardware_family_name(pyc_kernel_hardware_family family) {
    static const char* const names[] = {"any", "generic", "ada", "hopper", "cdna4"};
    if ((int)family < 0 || (int)family > (int)PYC_KERNEL_HARDWARE_CDNA4) {
        return "any";
    }
    return names[family];
}

static int entry_matches(const reg_entry* e, const char* op_key, pyc_backend backend) {
    return e->used && e->desc.backend == backend && strcmp(e->desc.op_key, op_key) == 0;
}

/* Per-mode weights: index 0 BALANCED, 1 MEMORY_FIRST, 2 UTILIZATION_FIRST. */
static int mode_index(pyc_objective_mode mode) {
    return (mode == PYC_MODE_MEMORY_FIRST) ? 1 : (mode == PYC_MODE_UTILIZATION_FIRST ? 2 : 0);
}

static double pressure_penalty_of(const pyc_kernel_desc* d, pyc_objective_mode mode, double pressure) {
    if (pressure <= 0.0 || mode == PYC_MODE_UTILIZATION_FIRST) {
        return 0.0;
    }
    return pressure * (double)(d->shared_mem_bytes / 1024U + (size_t)(d->reg_pressure_class * 8));
}

static double allocator_penalty_of(const pyc_kernel_desc* d, pyc_objective_mode mode,
                                   const pyc_kernel_coselect_context* ctx) {
    static const double w_pressure[3] = {7.0, 10.0, 3.0};
    static const double w_remat[3] = {10.0, 16.0, 5.0};
    static const double w_budget[3] = {90.0, 120.0, 45.0};
    const int mi = mode_index(mode);
    const double lds_kib = (double)d->shared_mem_bytes / 1024.0;
    const double rc = (double)d->reg_pressure_class;
    double p = 0.0;
    if (!ctx || mode == PYC_MODE_UTILIZATION_FIRST) {
        return 0.0;
    }
    if (ctx->pressure_events > 0) {
        p += (double)ctx->pressure_events * (w_pressure[mi] + 0.5 * lds_kib + 4.0 * rc);
    }
    if (ctx->rematerialized_tensors > 0) {
        p += (double)ctx->rematerialized_tensors * (w_remat[mi] + 0.35 * lds_kib + 3.0 * rc);
    }
    if (ctx->memory_budget_bytes > 0 && ctx->peak_bytes > ctx->memory_budget_bytes) {
        const double excess = (double)(ctx->peak_bytes - ctx->memory_budget_bytes) /
                              (double)ctx->memory_budget_bytes;
        p += excess * (w_budget[mi] + 1.5 * lds_kib + 12.0 * rc);
    }
    return p;
}

static double reuse_bonus_of(const pyc_kernel_desc* d, pyc_objective_mode mode,
                             const pyc_kernel_coselect_context* ctx) {
    static const double w_mode[3] = {24.0, 42.0, 10.0};
    double ratio, friendly;
    if (!ctx || ctx->total_requested_bytes == 0 || ctx->reused_allocations == 0 ||
        mode == PYC_MODE_UTILIZATION_FIRST) {
        return 0.0;
    }
    ratio = (double)ctx->reused_allocations / (double)(ctx->reused_allocations + ctx->pressure_events + 1U);
    friendly = 1.0 / (1.0 + (double)d->reg_pressure_class + (double)d->shared_mem_bytes / 32768.0);
    return ratio * friendly * w_mode[mode_index(mode)];
}

static double workload_affinity(const pyc_kernel_desc* d, const pyc_kernel_coselect_context* ctx) {
    if (!ctx || d->preferred_workload_family == PYC_KERNEL_WORKLOAD_ANY ||
        ctx->workload_family == PYC_KERNEL_WORKLOAD_ANY) {
        return 0.0;
    }
    return d->preferred_workload_family == ctx->workload_family ? 36.0 : -18.0;
}

static double hardware_affinity(const pyc_kernel_desc* d, const pyc_kernel_coselect_context* ctx) {
    if (!ctx || d->preferred_hardware_family == PYC_KERNEL_HARDWARE_ANY ||
        ctx->hardware_family == PYC_KERNEL_HARDWARE_ANY) {
        return 0.0;
    }
    if (d->preferred_hardware_family == ctx->hardware_family) {
        return 48.0;
    }
    if (ctx->hardware_family == PYC_KERNEL_HARDWARE_GENERIC &&
        d->preferred_hardware_family != PYC_KERNEL_HARDWARE_GENERIC) {
        return -8.0;
    }
    if (d->preferred_hardware_family == PYC_KERNEL_HARDWARE_GENERIC) {
        return 10.0;
    }
    return -24.0;
}

static double base_score_of(const reg_entry* e, pyc_objective_mode mode, double pressure, double* out_pen) {
    const pyc_kernel_desc* d = &e->desc;
    const double occ_w = mode == PYC_MODE_UTILIZATION_FIRST ? 12.0 : 6.0;
    const double measured = e->bench.best_time_ms;
    const double time_term = (measured <= 0.0 || measured == DBL_MAX) ? 0.0 : -100.0 * measured;
    const double pen = pressure_penalty_of(d, mode, pressure);
    if (out_pen) {
        *out_pen = pen;
    }
    return 100.0 * (double)d->priority + occ_w * d->estimated_occupancy +
           (d->tensor_core_eligible ? 25.0 : 0.0) + time_term - pen;
}

void pyc_kernel_registry_reset(void) {
    pyc_mutex_lock(&g_table_lock);
    memset(g_table, 0, sizeof(g_table));
    pyc_mutex_unlock(&g_table_lock);
}

int pyc_kernel_register(const pyc_kernel_desc* desc) {
    int rc = -1;
    size_t i;
    if (!desc || desc->op_key[0] == '\0') {
        return -1;
    }
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX; ++i) {
        if (!g_table[i].used) {
            memset(&g_table[i], 0, sizeof(g_table[i]));
            g_table[i].used = 1;
            g_table[i].desc = *desc;
            g_table[i].bench.best_time_ms = DBL_MAX;
            rc = 0;
            break;
        }
    }
    pyc_mutex_unlock(&g_table_lock);
    return rc;
}

int pyc_kernel_promote_symbol(const char* op_key, pyc_backend backend, const char* symbol) {
    size_t i;
    const int clear_only = !symbol || symbol[0] == '\0';
    int found = clear_only;
    if (!op_key) {
        return -1;
    }
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; !found && i < PYC_KERNEL_MAX; ++i) {
        if (entry_matches(&g_table[i], op_key, backend) && strcmp(g_table[i].desc.symbol, symbol) == 0) {
            found = 1;
        }
    }
    if (found) {
        for (i = 0; i < PYC_KERNEL_MAX; ++i) {
            if (entry_matches(&g_table[i], op_key, backend)) {
                g_table[i].promoted = !clear_only && strcmp(g_table[i].desc.symbol, symbol) == 0;
            }
        }
    }
    pyc_mutex_unlock(&g_table_lock);
    return found ? 0 : -1;
}

int pyc_kernel_promoted_symbol(const char* op_key, pyc_backend backend, char* out_symbol,
                               size_t out_symbol_size) {
    size_t i;
    int rc = -1;
    if (!op_key || !out_symbol || out_symbol_size == 0) {
        return -1;
    }
    out_symbol[0] = '\0';
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX; ++i) {
        if (entry_matches(&g_table[i], op_key, backend) && g_table[i].promoted) {
            strncpy(out_symbol, g_table[i].desc.symbol, out_symbol_size - 1);
            out_symbol[out_symbol_size - 1] = '\0';
            rc = 0;
            break;
        }
    }
    pyc_mutex_unlock(&g_table_lock);
    return rc;
}

int pyc_kernel_select(const char* op_key, pyc_backend backend, pyc_kernel_desc* out) {
    return pyc_kernel_select_with_policy(op_key, backend, PYC_MODE_BALANCED, 0.0, out, NULL);
}

/* Shared best-candidate scan. ctx == NULL and joint == 0 gives the plain
 * policy score; joint == 1 gives the allocator-aware joint score. */
static int scan_best(const char* op_key, pyc_backend backend, pyc_objective_mode mode,
                     double pressure, const pyc_kernel_coselect_context* ctx, int joint,
                     pyc_kernel_desc* out, pyc_kernel_selection_trace* trace) {
    size_t i;
    int have = 0;
    size_t considered = 0;
    double best = 0.0, best_pen = 0.0, best_alloc = 0.0, best_reuse = 0.0, best_occ = 0.0;
    pyc_kernel_desc pick;
    memset(&pick, 0, sizeof(pick));
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX; ++i) {
        const reg_entry* e = &g_table[i];
        double pen = 0.0, alloc = 0.0, reuse = 0.0, s;
        if (!entry_matches(e, op_key, backend)) {
            continue;
        }
        considered++;
        s = base_score_of(e, mode, joint ? (ctx ? ctx->pressure_score : 0.0) : pressure, &pen);
        if (joint) {
            alloc = allocator_penalty_of(&e->desc, mode, ctx);
            reuse = reuse_bonus_of(&e->desc, mode, ctx);
            s = s - alloc + reuse + workload_affinity(&e->desc, ctx) + hardware_affinity(&e->desc, ctx);
        }
        if (!have || s > best || (s == best && strcmp(e->desc.symbol, pick.symbol) < 0)) {
            have = 1;
            best = s;
            best_pen = pen;
            best_alloc = alloc;
            best_reuse = reuse;
            best_occ = e->desc.estimated_occupancy;
            pick = e->desc;
        }
    }
    pyc_mutex_unlock(&g_table_lock);
    if (!have) {
        return -1;
    }
    *out = pick;
    if (trace) {
        trace->selected_score = best;
        trace->selected_estimated_utilization = best_occ;
        trace->pressure_penalty = best_pen;
        trace->allocator_penalty = best_alloc;
        trace->reuse_bonus = best_reuse;
        trace->candidates_considered = joint ? considered : 0;
    }
    return 0;
}

int pyc_kernel_select_with_policy(const char* op_key, pyc_backend backend, pyc_objective_mode mode,
                                  double pressure_score, pyc_kernel_desc* out,
                                  pyc_kernel_selection_trace* trace) {
    if (!op_key || !out) {
        return -1;
    }
    return scan_best(op_key, backend, mode, pressure_score, NULL, 0, out, trace);
}

int pyc_kernel_coselect_with_context(const char* op_key, pyc_backend backend, pyc_objective_mode mode,
                                     const pyc_kernel_coselect_context* context, pyc_kernel_desc* out,
                                     pyc_kernel_selection_trace* trace) {
    if (!op_key || !out) {
        return -1;
    }
    return scan_best(op_key, backend, mode, 0.0, context, 1, out, trace);
}

int pyc_kernel_benchmark_update_symbol(const char* op_key, pyc_backend backend, const char* symbol,
                                       double time_ms) {
    size_t i;
    int hit = 0;
    if (!op_key) {
        return -1;
    }
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX; ++i) {
        reg_entry* e = &g_table[i];
        if (!entry_matches(e, op_key, backend)) {
            continue;
        }
        if (symbol && symbol[0] != '\0' && strcmp(e->desc.symbol, symbol) != 0) {
            continue;
        }
        e->bench.considered++;
        if (time_ms < e->bench.best_time_ms) {
            e->bench.best_time_ms = time_ms;
            e->bench.selected++;
        }
        hit = 1;
    }
    pyc_mutex_unlock(&g_table_lock);
    return hit ? 0 : -1;
}

int pyc_kernel_benchmark_update(const char* op_key, pyc_backend backend, double time_ms) {
    return pyc_kernel_benchmark_update_symbol(op_key, backend, NULL, time_ms);
}

void pyc_kernel_benchmark_read(const char* op_key, pyc_backend backend, pyc_kernel_benchmark* out) {
    size_t i;
    if (!out) {
        return;
    }
    memset(out, 0, sizeof(*out));
    if (!op_key) {
        return;
    }
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX; ++i) {
        const reg_entry* e = &g_table[i];
        if (!entry_matches(e, op_key, backend)) {
            continue;
        }
        out->considered += e->bench.considered;
        out->selected += e->bench.selected;
        if (out->best_time_ms == 0.0 || e->bench.best_time_ms < out->best_time_ms) {
            out->best_time_ms = e->bench.best_time_ms;
        }
    }
    pyc_mutex_unlock(&g_table_lock);
}

size_t pyc_kernel_collect(const char* op_key, pyc_backend backend, pyc_kernel_desc* out_descs,
                          size_t out_capacity) {
    size_t i, n = 0;
    if (!op_key || !out_descs || out_capacity == 0) {
        return 0;
    }
    pyc_mutex_lock(&g_table_lock);
    for (i = 0; i < PYC_KERNEL_MAX && n < out_capacity; ++i) {
        size_t at;
        if (!entry_matches(&g_table[i], op_key, backend)) {
            continue;
        }
        /* insertion into lexical order by symbol */
        at = n;
        while (at > 0 && strcmp(g_table[i].desc.symbol, out_descs[at - 1].symbol) < 0) {
            out_descs[at] = out_descs[at - 1];
            at--;
        }
        out_descs[at] = g_table[i].desc;
        n++;
    }
    pyc_mutex_unlock(&g_table_lock);
    return n;
}
