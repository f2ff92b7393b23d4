/*
 * dispatch.c -- the kernel dispatch table (see sllm_kdispatch.h).
 *
 * One built-in row, gfx950. Selection happens once, at model load, on the
 * loading thread (src/forward.c:324-334); the hot calls read the installed
 * row without locking, as the reference reads g_dot (src/i2s_gemm.c:239-258).
 */
#define _POSIX_C_SOURCE 200809L

#include <saphira_amd/sllm_kdispatch.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifndef SLLM_GFX950_DEVICE
#define SLLM_GFX950_DEVICE 0
#endif

static int gfx950_open(void) { return sllm_gfx950_open(SLLM_GFX950_DEVICE); }

/* sllm_gemv hands over whole matrices (src/forward.c:196-205): the first call
 * on a matrix uploads it, so the loader need not register anything */
static void gfx950_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q, int32_t *rows_out) {
    if (w != NULL && q != NULL && rows_out != NULL && n_rows > 0 && n >= SLLM_GFX950_QK) {
        const int st = sllm_gfx950_tensor_acquire(w, n_rows, n);
        if (st != SLLM_GFX950_OK) {
            fprintf(stderr, "sllm_kdispatch_gemv: the gfx950 row cannot take the weights at %p (%d): %s\n",
                    (const void *) w, st, sllm_gfx950_last_error());
            abort();
        }
    }
    sllm_gfx950_i2s_gemv(w, n_rows, n, q, rows_out);
}

static void gfx950_release(void) {
    const int st = sllm_gfx950_tensor_release_acquired();
    if (st != SLLM_GFX950_OK && st != SLLM_GFX950_ERR_NO_DEVICE) {
        fprintf(stderr, "sllm_kdispatch_release: %s\n", sllm_gfx950_last_error());
    }
}

static const sllm_kernel_row k_gfx950_row = {
    "gfx950", 100, gfx950_open,
    sllm_gfx950_i2s_quant_act, sllm_gfx950_i2s_dot, gfx950_gemv, gfx950_release,
};

static sllm_kernel_row g_rows[SLLM_KDISPATCH_MAX_ROWS] = { k_gfx950_row };
static size_t g_n_rows = 1;
static const sllm_kernel_row *g_installed = NULL;

int sllm_kdispatch_register(const sllm_kernel_row *row) {
    if (row == NULL || row->name == NULL || row->quant_act == NULL || row->dot == NULL ||
        row->gemv == NULL) {
        return SLLM_GFX950_ERR_ARG;
    }
    if (g_n_rows == SLLM_KDISPATCH_MAX_ROWS) return SLLM_GFX950_ERR_ARG;
    for (size_t i = 0; i < g_n_rows; ++i) {
        if (strcmp(g_rows[i].name, row->name) == 0) return SLLM_GFX950_ERR_ARG;
    }
    g_rows[g_n_rows++] = *row;
    return SLLM_GFX950_OK;
}

size_t sllm_kdispatch_count(void) { return g_n_rows; }

const sllm_kernel_row *sllm_kdispatch_row(size_t i) { return i < g_n_rows ? &g_rows[i] : NULL; }

static int try_open(const sllm_kernel_row *r) { return r->open ? r->open() : SLLM_GFX950_OK; }

int sllm_kdispatch_select(const char *name) {
    if (name == NULL) return SLLM_GFX950_ERR_ARG;
    if (strcmp(name, "auto") == 0) {
        /* highest priority first; ties keep registration order */
        int tried[SLLM_KDISPATCH_MAX_ROWS] = { 0 };
        int last = SLLM_GFX950_ERR_NO_DEVICE;
        for (size_t n = 0; n < g_n_rows; ++n) {
            size_t best = g_n_rows;
            for (size_t i = 0; i < g_n_rows; ++i) {
                if (!tried[i] && (best == g_n_rows || g_rows[i].priority > g_rows[best].priority)) best = i;
            }
            tried[best] = 1;
            last = try_open(&g_rows[best]);
            if (last == SLLM_GFX950_OK) {
                g_installed = &g_rows[best];
                return SLLM_GFX950_OK;
            }
        }
        return last;
    }
    for (size_t i = 0; i < g_n_rows; ++i) {
        if (strcmp(g_rows[i].name, name) == 0) {
            const int st = try_open(&g_rows[i]);
            if (st == SLLM_GFX950_OK) g_installed = &g_rows[i];
            return st;
        }
    }
    return SLLM_GFX950_ERR_ARG;
}

const sllm_kernel_row *sllm_kdispatch_installed(void) { return g_installed; }

const char *sllm_kdispatch_installed_name(void) { return g_installed ? g_installed->name : "none"; }

void sllm_kdispatch_reset(void) { g_installed = NULL; }

static const sllm_kernel_row *need_row(const char *fn) {
    if (g_installed == NULL) {
        fprintf(stderr, "sllm_kdispatch: %s called with no kernel row installed "
                        "(call sllm_kdispatch_select at model load)\n", fn);
        abort();
    }
    return g_installed;
}

void sllm_kdispatch_quant_act(const float *x, size_t n, int8_t *q_out, sllm_gfx950_act *out) {
    need_row("sllm_kdispatch_quant_act")->quant_act(x, n, q_out, out);
}

int32_t sllm_kdispatch_dot(const uint8_t *w, const int8_t *q, size_t n) {
    return need_row("sllm_kdispatch_dot")->dot(w, q, n);
}

void sllm_kdispatch_gemv(const uint8_t *w, size_t n_rows, size_t n, const int8_t *q,
                         int32_t *rows_out) {
    need_row("sllm_kdispatch_gemv")->gemv(w, n_rows, n, q, rows_out);
}

void sllm_kdispatch_release(void) {
    if (g_installed != NULL && g_installed->release != NULL) g_installed->release();
}
