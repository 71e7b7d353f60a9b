/* runtime_allocator.c — first-fit lifetime-reuse offset planner.
 *
 * Behaviour of reference src/compiler/runtime/runtime_allocator.c:6-237:
 * requests are placed in order; a request reuses the offset of an earlier,
 * at-least-as-large request when no request already at that offset is live
 * during its [start_step, end_step]; otherwise it is appended at the aligned
 * peak. Over a memory budget the plan records one pressure event, a pressure
 * score of excess/budget, and estimates rematerialisation relief greedily by
 * bytes-per-lifetime-step (all of the excess in MEMORY_FIRST, half and a single
 * tensor in BALANCED, none in UTILIZATION_FIRST). On the GPU backend these
 * offsets are what the HIP workspace would sub-allocate; the figures feed the
 * kernel registry's allocator-aware scoring. */
#include "pyc/runtime_allocator.h"

#include <string.h>

static int live_together(const pyc_alloc_request* a, const pyc_alloc_request* b) {
    return a->start_step <= b->end_step && b->start_step <= a->end_step;
}

static size_t round_up(size_t v, size_t a) {
    if (a == 0) {
        a = 1;
    }
    return (v + a - 1) / a * a;
}

void pyc_alloc_plan_init(pyc_alloc_plan* plan) {
    if (plan) {
        memset(plan, 0, sizeof(*plan));
    }
}

int pyc_alloc_plan_add_request(pyc_alloc_plan* plan, pyc_alloc_request req) {
    if (!plan || plan->request_count >= PYC_ALLOC_MAX_REQUESTS || req.size_bytes == 0 ||
        req.end_step < req.start_step) {
        return -1;
    }
    plan->requests[plan->request_count++] = req;
    return 0;
}

int pyc_alloc_plan_build(pyc_alloc_plan* plan) {
    return pyc_alloc_plan_build_with_mode(plan, PYC_MODE_BALANCED, 0);
}

/* bytes freed per step of lifetime if the tensor were recomputed instead of kept */
static size_t remat_gain(const pyc_alloc_request* r, size_t* span_out) {
    const size_t span = r->end_step >= r->start_step ? (size_t)(r->end_step - r->start_step + 1) : 0;
    *span_out = span;
    if (r->size_bytes == 0) {
        return 0;
    }
    return span <= 1 ? r->size_bytes : r->size_bytes / span;
}

static size_t relieve(pyc_alloc_plan* plan, pyc_objective_mode mode, size_t target) {
    size_t gain[PYC_ALLOC_MAX_REQUESTS];
    size_t span[PYC_ALLOC_MAX_REQUESTS];
    size_t n = 0, i, got = 0;
    for (i = 0; i < plan->request_count; ++i) {
        size_t s;
        const size_t g = remat_gain(&plan->requests[i], &s);
        if (g) {
            gain[n] = g;
            span[n] = s;
            n++;
        }
    }
    while (n > 0 && got < target) {
        size_t best = 0;
        for (i = 1; i < n; ++i) {
            const size_t di = span[i] ? span[i] : 1;
            const size_t db = span[best] ? span[best] : 1;
            if (gain[i] * db > gain[best] * di) {
                best = i;
            }
        }
        got += gain[best];
        plan->rematerialized_tensors++;
        plan->rematerialized_bytes += gain[best];
        gain[best] = gain[n - 1];
        span[best] = span[n - 1];
        n--;
        if (mode == PYC_MODE_BALANCED) {
            break;
        }
    }
    return got;
}

int pyc_alloc_plan_build_with_mode(pyc_alloc_plan* plan, pyc_objective_mode mode, size_t budget) {
    size_t i, j, k;
    if (!plan) {
        return -1;
    }
    plan->peak_bytes = 0;
    plan->reused_allocations = 0;
    plan->allocation_events = 0;
    plan->overlap_pairs_observed = 0;
    plan->largest_allocation_bytes = 0;
    plan->rematerialized_tensors = 0;
    plan->rematerialized_bytes = 0;
    plan->pressure_events = 0;
    plan->pressure_score = 0.0;
    for (i = 0; i < plan->request_count; ++i) {
        const pyc_alloc_request* cur = &plan->requests[i];
        int placed = 0;
        for (j = 0; j < i; ++j) {
            plan->overlap_pairs_observed += live_together(&plan->requests[j], cur) ? 1u : 0u;
        }
        for (j = 0; j < i && !placed; ++j) {
            int clash = 0;
            if (plan->requests[j].size_bytes < cur->size_bytes) {
                continue;
            }
            for (k = 0; k < i && !clash; ++k) {
                clash = plan->offsets[k] == plan->offsets[j] && live_together(&plan->requests[k], cur);
            }
            if (!clash) {
                plan->offsets[i] = plan->offsets[j];
                plan->reused_allocations++;
                placed = 1;
            }
        }
        if (!placed) {
            plan->offsets[i] = round_up(plan->peak_bytes, cur->alignment);
            plan->peak_bytes = plan->offsets[i] + cur->size_bytes;
            plan->allocation_events++;
        }
        if (cur->size_bytes > plan->largest_allocation_bytes) {
            plan->largest_allocation_bytes = cur->size_bytes;
        }
    }
    if (budget > 0 && plan->peak_bytes > budget) {
        const size_t excess = plan->peak_bytes - budget;
        size_t target = 0, got;
        plan->pressure_events = 1;
        plan->pressure_score = (double)excess / (double)budget;
        if (mode == PYC_MODE_MEMORY_FIRST) {
            target = excess;
        } else if (mode == PYC_MODE_BALANCED) {
            target = excess / 2 ? excess / 2 : 1;
        }
        got = relieve(plan, mode, target);
        if (got > 0) {
            plan->peak_bytes = got >= excess ? budget : plan->peak_bytes - got;
        }
    }
    return 0;
}

void pyc_alloc_plan_stats(const pyc_alloc_plan* plan, pyc_alloc_stats* stats) {
    size_t i;
    if (!plan || !stats) {
        return;
    }
    memset(stats, 0, sizeof(*stats));
    stats->peak_bytes = plan->peak_bytes;
    stats->reused_allocations = plan->reused_allocations;
    stats->allocation_events = plan->allocation_events;
    stats->overlap_pairs_observed = plan->overlap_pairs_observed;
    stats->largest_allocation_bytes = plan->largest_allocation_bytes;
    stats->rematerialized_tensors = plan->rematerialized_tensors;
    stats->rematerialized_bytes = plan->rematerialized_bytes;
    stats->pressure_events = plan->pressure_events;
    stats->pressure_score = plan->pressure_score;
    for (i = 0; i < plan->request_count; ++i) {
        stats->total_requested_bytes += plan->requests[i].size_bytes;
    }
}
