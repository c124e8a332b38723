/*
 * kyro_testing.h — test-only controls of libkyro_verify. No counterpart in the reference: these
 * exist so that the library's own tests can force conditions a correct caller never produces.
 * A production caller never calls them; a process that does not call them behaves exactly as
 * if they did not exist (no environment variable or other implicit input is read).
 */
#ifndef KYRO_TESTING_H
#define KYRO_TESTING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Caps the partial-state slots a balanced-schedule kyro_paged_attention_mq call sizes at `cap`
 * (process-wide; 0, the initial state, sizes the full bound). With a cap below what the plan
 * needs, the device plan latches an error and runs no item, and the next kyro_sync returns
 * KYRO_EINVAL. Returns the previous cap. */
int64_t kyro_testing_set_plan_slot_cap(int64_t cap);

#ifdef __cplusplus
}
#endif

#endif /* KYRO_TESTING_H */
