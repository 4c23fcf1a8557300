/*
 * Span recording with Chrome-Tracing JSON output: the reference's trace
 * interface (pitorch/profiler/trace.h:21-101, trace.c:20-98) for the host
 * layer.  Host spans are timed with gettimeofday like the reference's Mac
 * build; a traced pt_train_step appends the device step's spans, timed
 * with HIP events on the GPU, under the same names.
 */
#include <stdio.h>
#include <string.h>
#include <sys/time.h>

#include "pt.h"

uint32_t pt_time_us(void) {
    struct timeval tv;
    gettimeofday(&tv, NULL);
    return (uint32_t)((uint64_t)tv.tv_sec * 1000000u + (uint64_t)tv.tv_usec);
}

size_t pt_trace_size(void) { return sizeof(pt_trace_t); }

void pt_trace_init(pt_trace_t *t) {
    if (!t) return;
    memset(t, 0, sizeof(*t));
    t->enabled = 1;
}

void pt_trace_begin(pt_trace_t *t, const char *name, const char *cat, int layer) {
    if (!t || !t->enabled || t->depth >= PT_TRACE_MAX_DEPTH) return;
    t->stack[t->depth].name = name;
    t->stack[t->depth].cat = cat;
    t->stack[t->depth].layer = (int8_t)layer;
    t->stack[t->depth].ts_us = pt_time_us();
    t->depth++;
}

/* Record one finished span (also used for the device step's spans). */
void pt_trace_add(pt_trace_t *t, const char *name, const char *cat, int layer, int depth, uint32_t ts_us,
                  uint32_t dur_us) {
    if (!t || !t->enabled || t->count >= PT_TRACE_MAX_EVENTS) return;
    pt_trace_event_t *e = &t->events[t->count++];
    e->name = name;
    e->cat = cat;
    e->ts_us = ts_us;
    e->dur_us = dur_us;
    e->layer = (int8_t)layer;
    e->depth = (int8_t)depth;
    e->hw_cycles = 0;
    e->hw_stall = 0;
}

void pt_trace_end(pt_trace_t *t) {
    if (!t || !t->enabled || t->depth <= 0) return;
    const uint32_t now = pt_time_us();
    t->depth--;
    pt_trace_add(t, t->stack[t->depth].name, t->stack[t->depth].cat, t->stack[t->depth].layer, t->depth,
                 t->stack[t->depth].ts_us, now - t->stack[t->depth].ts_us);
}

void pt_trace_reset(pt_trace_t *t) {
    if (!t) return;
    t->count = 0;
    t->depth = 0;
}

/* Chrome Tracing "complete" events; a layer span is named L<layer>_<name>. */
void pt_trace_write_json(const pt_trace_t *t, const char *path) {
    if (!t || t->count == 0 || !path) return;
    FILE *f = fopen(path, "w");
    if (!f) return;
    fputs("[\n", f);
    for (int i = 0; i < t->count; i++) {
        const pt_trace_event_t *e = &t->events[i];
        if (i) fputs(",\n", f);
        if (e->layer >= 0) fprintf(f, "{\"name\":\"L%d_%s\"", e->layer, e->name);
        else fprintf(f, "{\"name\":\"%s\"", e->name);
        fprintf(f, ",\"cat\":\"%s\",\"ph\":\"X\",\"ts\":%u,\"dur\":%u,\"pid\":0,\"tid\":0", e->cat, e->ts_us,
                e->dur_us);
        if (e->hw_cycles || e->hw_stall)
            fprintf(f, ",\"args\":{\"qpu_exec\":%u,\"tmu_stall\":%u}", e->hw_cycles, e->hw_stall);
        fputc('}', f);
    }
    fputs("\n]\n", f);
    fclose(f);
}

void pt_trace_write_meta(const char *path, const char *name, const char *model, int dim, int layers, int vocab,
                         const char *device, int num_qpus, int steps, float lr, float final_loss,
                         float total_time_s, const char *notes) {
    if (!path) return;
    FILE *f = fopen(path, "w");
    if (!f) return;
    fprintf(f, "{\n  \"name\": \"%s\",\n  \"model\": \"%s\",\n", name ? name : "", model ? model : "");
    fprintf(f, "  \"dim\": %d, \"layers\": %d, \"vocab\": %d,\n", dim, layers, vocab);
    fprintf(f, "  \"device\": \"%s\",\n  \"num_qpus\": %d,\n  \"steps\": %d,\n", device ? device : "", num_qpus, steps);
    fprintf(f, "  \"lr\": %.6f,\n  \"final_loss\": %.6f,\n  \"total_time_s\": %.1f,\n", lr, final_loss, total_time_s);
    fprintf(f, "  \"notes\": \"%s\"\n}\n", notes ? notes : "");
    fclose(f);
}
