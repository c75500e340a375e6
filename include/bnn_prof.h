/* bnn_prof.h - per-op profiler API of libbnn_hip.so.
 *
 * Same entry points and meaning as the reference's csrc/bnn_prof.h:13-17
 * (used by its csrc/main.c).  prof_now() is host CLOCK_MONOTONIC seconds.
 * Records come from the GPU forward when bnn_prof_enable(1) is set: one row
 * per kernel with its hipEvent-measured time, labelled like the reference's
 * per-op rows (enc1.conv1, enc2.c1, ...); prof_report() is silent when there
 * are none.
 */
#ifndef BNN_PROF_H
#define BNN_PROF_H
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

double prof_now(void);
void   prof_reset(void);
void   prof_add(const char *label, const char *optype,
                double out_elems, double taps, double sec);
void   prof_report(FILE *out);

#ifdef __cplusplus
}
#endif
#endif
