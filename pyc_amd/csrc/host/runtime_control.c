/* runtime_control.c — objective-mode controller ticked once per pyc_run_model.
 *
 * Behaviour of reference src/compiler/runtime/runtime_control.c:5-156: default
 * rails (dwell 4, cooldown 2, 2 consecutive breach windows, latency +8%,
 * throughput -5%, pressure 0.20 / 1 event / 4 rematerialisations), breach
 * precedence runtime-error > pressure > latency > throughput, hard rollback to
 * BALANCED after the configured number of consecutive breaches, otherwise an
 * auto-switch to the recommended mode once dwell and cooldown allow. */
#include "pyc/runtime_control.h"

#include <string.h>

void pyc_runtime_rails_default(pyc_runtime_rails* rails) {
    if (!rails) {
        return;
    }
    memset(rails, 0, sizeof(*rails));
    rails->enable_auto_switch = 1;
    rails->enable_hard_rollback = 1;
    rails->dwell_steps = 4;
    rails->cooldown_steps = 2;
    rails->consecutive_breach_windows = 2;
    rails->latency_regression_threshold = 0.08;
    rails->throughput_regression_threshold = 0.05;
    rails->pressure_score_threshold = 0.20;
    rails->pressure_events_threshold = 1;
    rails->rematerialized_tensors_threshold = 4;
}

void pyc_runtime_controller_init(pyc_runtime_controller* c, pyc_objective_mode initial_mode) {
    if (!c) {
        return;
    }
    memset(c, 0, sizeof(*c));
    c->current_mode = initial_mode;
    c->recommended_mode = initial_mode;
    c->recommendation_reason = PYC_ROLLBACK_NONE;
    c->last_stable_mode = initial_mode;
}

/* Which rail (if any) the window breaches, and the mode it recommends. */
static int classify_window(const pyc_runtime_controller* c, const pyc_runtime_rails* r,
                           const pyc_runtime_window_metrics* m, pyc_objective_mode* mode,
                           pyc_rollback_reason* reason) {
    const int pressure = m->pressure_score > r->pressure_score_threshold ||
                         m->pressure_events >= r->pressure_events_threshold ||
                         m->rematerialized_tensors >= r->rematerialized_tensors_threshold;
    const int latency = m->baseline_p95_ms > 0.0 &&
                        m->observed_p95_ms > m->baseline_p95_ms * (1.0 + r->latency_regression_threshold);
    const int throughput = m->baseline_throughput > 0.0 &&
                           m->observed_throughput < m->baseline_throughput * (1.0 - r->throughput_regression_threshold);
    *mode = c->current_mode;
    *reason = PYC_ROLLBACK_NONE;
    if (m->runtime_error) {
        *mode = PYC_MODE_BALANCED;
        *reason = PYC_ROLLBACK_RUNTIME_ERROR;
    } else if (pressure) {
        *mode = PYC_MODE_MEMORY_FIRST;
        *reason = PYC_ROLLBACK_PRESSURE;
    } else if (latency) {
        *mode = PYC_MODE_BALANCED;
        *reason = PYC_ROLLBACK_LATENCY;
    } else if (throughput) {
        *mode = PYC_MODE_UTILIZATION_FIRST;
        *reason = PYC_ROLLBACK_THROUGHPUT;
    } else {
        if (c->current_mode != PYC_MODE_BALANCED) {
            *mode = PYC_MODE_BALANCED; /* healthy window: drift back to balanced */
        }
        return 0;
    }
    return 1;
}

int pyc_runtime_controller_observe(pyc_runtime_controller* c, const pyc_runtime_rails* r,
                                   const pyc_runtime_window_metrics* m, pyc_objective_mode* out_mode,
                                   pyc_rollback_reason* out_reason) {
    pyc_objective_mode rec;
    pyc_rollback_reason why;
    int breached;
    if (!c || !r || !m || !out_mode || !out_reason) {
        return -1;
    }
    c->steps_in_mode++;
    if (c->cooldown_remaining > 0) {
        c->cooldown_remaining--;
    }
    breached = classify_window(c, r, m, &rec, &why);
    c->recommended_mode = rec;
    c->recommendation_reason = why;
    c->consecutive_breaches = breached ? c->consecutive_breaches + 1 : 0;
    if (r->enable_hard_rollback && c->consecutive_breaches >= r->consecutive_breach_windows) {
        c->last_rollback_reason = why;
        c->rollback_count++;
        c->current_mode = PYC_MODE_BALANCED;
        c->last_stable_mode = PYC_MODE_BALANCED;
        c->steps_in_mode = 0;
        c->cooldown_remaining = r->cooldown_steps;
        c->consecutive_breaches = 0;
    } else if (r->enable_auto_switch && c->cooldown_remaining == 0 && c->steps_in_mode >= r->dwell_steps &&
               rec != c->current_mode) {
        c->current_mode = rec;
        c->last_stable_mode = rec;
        c->steps_in_mode = 0;
        c->cooldown_remaining = r->cooldown_steps;
        c->consecutive_breaches = 0;
    }
    *out_mode = c->current_mode;
    *out_reason = c->last_rollback_reason;
    return 0;
}
