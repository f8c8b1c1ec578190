/*
 * pa_decode_timeline.h - phase timeline of the decode kernel (measurement
 * build only).
 *
 * libpa_decode_tl.so is the same source as libpa_decode.so (pa_decode.h),
 * compiled with -DPAD_TIMELINE: thread 0 of every workgroup stores
 * s_memrealtime stamps (a 100 MHz constant clock shared by all CUs) at
 * fixed points of the kernel.  The stamps feed the per-phase time budget
 * (profile_run --timeline).  The product path never loads this library, and
 * libpa_decode.so exports none of these functions.
 *
 * No counterpart in the reference, whose phase split came from Nsight
 * Compute profiles of its two kernels (profiles/notes.md:848-883).
 *
 * Buffer layout: [PAD_TL_LAUNCHES][PAD_TL_MAX_GROUPS][PAD_TL_SLOTS] uint64.
 * Launch n (counted from the last pad_timeline_reset()) writes ring entry
 * n % PAD_TL_LAUNCHES; workgroup L (linear index of the launch grid, x
 * fastest) writes row L.  A slot a workgroup never reaches stays 0.
 */
#ifndef PA_DECODE_TIMELINE_H_
#define PA_DECODE_TIMELINE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PAD_TL_LAUNCHES 4
#define PAD_TL_MAX_GROUPS 16384
#define PAD_TL_SLOTS 8

/* Slots of one workgroup's row. */
#define PAD_TL_ENTRY 0      /* first instruction                              */
#define PAD_TL_ITEM 1       /* work item known (page range, unit)             */
#define PAD_TL_LOOP_END 2   /* every wave's streaming loop done (barrier)     */
#define PAD_TL_PUBLISHED 3  /* partial stores complete at device scope, or
                               the output rows written (one-split unit)       */
#define PAD_TL_ARRIVED 4    /* unit arrival atomic returned                   */
#define PAD_TL_MERGED 5     /* the last arrival's merge written               */
#define PAD_TL_EXIT 6       /* last stamp before the workgroup ends           */
#define PAD_TL_INFO 7       /* not a time: bits 0-31 item slot (or -1),
                               32-35 XCC id, 40-47 flags (PAD_TL_F_*)         */
#define PAD_TL_F_NO_ITEM 1
#define PAD_TL_F_SINGLE 2   /* the unit had one item: no partials, no merge  */
#define PAD_TL_F_MERGER 4   /* last arrival of its unit                       */
#define PAD_TL_F_GROUP 8    /* last arrival of a two-level merge group        */

/* Copy the stamp buffer (at most `bytes`) to host memory; synchronous. */
int pad_timeline_read(void* host, size_t bytes);

/* Zero the stamp buffer and restart the launch count at 0; synchronous. */
int pad_timeline_reset(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* PA_DECODE_TIMELINE_H_ */
