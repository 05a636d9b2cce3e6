/* checkpoint.c -- weights-only (CKPT) and full training-state (CKTR)
 * checkpoints in the reference's on-disk format (src/checkpoint.c:1-136), so a
 * run can resume from a file written by either implementation:
 *
 *   u32 magic ("CKPT" 0x434B5054 or "CKTR" 0x434B5452), native endianness
 *   CKTR only: i32 step, i32 adam_t
 *   then per ParamList (CKPT: params; CKTR: params, EMA shadow, Adam m, Adam v):
 *     i32 count, count x i32 sizes, then the float32 payloads in list order.
 *
 * Lists are ParamList-ordered per-tensor buffers (optimizer_moment_lists,
 * ema_shadow_list), the order the fused multi-tensor optimizer also keeps.
 * Return codes as the reference's: 0 ok, -1 open failed, -2 bad magic or
 * short file, -3 tensor count mismatch, -4 tensor size mismatch.  A load
 * validates every list header before it writes any device memory of that list.
 */
#include <string.h>

#include "nn_modules.h"

#define NN_CKPT_MAGIC 0x434B5054u       /* "CKPT": weights only */
#define NN_CKPT_TRAIN_MAGIC 0x434B5452u /* "CKTR": full training state */

static int ck_read(void* dst, size_t size, size_t n, FILE* f)
{
    return fread(dst, size, n, f) == n ? 0 : -1;
}

static int ck_write(const void* src, size_t size, size_t n, FILE* f)
{
    return fwrite(src, size, n, f) == n ? 0 : -1;
}

static int write_list(FILE* f, const ParamList* pl)
{
    if (ck_write(&pl->count, sizeof(int), 1, f)) return -1;
    for (int i = 0; i < pl->count; ++i)
        if (ck_write(&pl->items[i].size, sizeof(int), 1, f)) return -1;
    size_t cap = 0;
    float* buf = NULL;
    for (int i = 0; i < pl->count; ++i) {
        const size_t n = (size_t)pl->items[i].size;
        if (n > cap) {
            free(buf);
            buf = (float*)malloc(n * sizeof(float));
            cap = n;
        }
        NN_HIP_CHECK(hipMemcpy(buf, pl->items[i].param, n * sizeof(float), hipMemcpyDeviceToHost));
        if (ck_write(buf, sizeof(float), n, f)) {
            free(buf);
            return -1;
        }
    }
    free(buf);
    return 0;
}

static int read_list(FILE* f, ParamList* pl)
{
    int count;
    if (ck_read(&count, sizeof(int), 1, f)) return -2;
    if (count != pl->count) {
        fprintf(stderr, "checkpoint: param count mismatch (file=%d, model=%d)\n", count, pl->count);
        return -3;
    }
    for (int i = 0; i < count; ++i) {
        int size;
        if (ck_read(&size, sizeof(int), 1, f)) return -2;
        if (size != pl->items[i].size) {
            fprintf(stderr, "checkpoint: param %d size mismatch (file=%d, model=%d)\n", i, size,
                pl->items[i].size);
            return -4;
        }
    }
    size_t cap = 0;
    float* buf = NULL;
    for (int i = 0; i < count; ++i) {
        const size_t n = (size_t)pl->items[i].size;
        if (n > cap) {
            free(buf);
            buf = (float*)malloc(n * sizeof(float));
            cap = n;
        }
        if (ck_read(buf, sizeof(float), n, f)) {
            free(buf);
            return -2;
        }
        NN_HIP_CHECK(hipMemcpy(pl->items[i].param, buf, n * sizeof(float), hipMemcpyHostToDevice));
    }
    free(buf);
    return 0;
}

int checkpoint_save(const char* path, const ParamList* pl)
{
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    const unsigned magic = NN_CKPT_MAGIC;
    int rc = ck_write(&magic, sizeof magic, 1, f) ? -1 : write_list(f, pl);
    if (fclose(f) && !rc) rc = -1;
    return rc;
}

int checkpoint_load(const char* path, ParamList* pl)
{
    FILE* f = fopen(path, "rb");
    if (!f) return -1;
    unsigned magic;
    int rc = (ck_read(&magic, sizeof magic, 1, f) || magic != NN_CKPT_MAGIC) ? -2 : read_list(f, pl);
    fclose(f);
    return rc;
}

int checkpoint_save_training(const char* path, int step, int adam_t, const ParamList* params,
    const ParamList* ema_shadow, const ParamList* adam_m, const ParamList* adam_v)
{
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    const unsigned magic = NN_CKPT_TRAIN_MAGIC;
    int rc = (ck_write(&magic, sizeof magic, 1, f) || ck_write(&step, sizeof(int), 1, f) ||
                 ck_write(&adam_t, sizeof(int), 1, f)) ? -1 : 0;
    const ParamList* lists[4] = {params, ema_shadow, adam_m, adam_v};
    for (int k = 0; k < 4 && !rc; ++k) rc = write_list(f, lists[k]);
    if (fclose(f) && !rc) rc = -1;
    return rc;
}

int checkpoint_load_training(const char* path, int* step, int* adam_t, ParamList* params,
    ParamList* ema_shadow, ParamList* adam_m, ParamList* adam_v)
{
    FILE* f = fopen(path, "rb");
    if (!f) return -1;
    unsigned magic;
    int rc = 0;
    if (ck_read(&magic, sizeof magic, 1, f) || magic != NN_CKPT_TRAIN_MAGIC || ck_read(step, sizeof(int), 1, f) ||
        ck_read(adam_t, sizeof(int), 1, f))
        rc = -2;
    ParamList* lists[4] = {params, ema_shadow, adam_m, adam_v};
    for (int k = 0; k < 4 && !rc; ++k) rc = read_list(f, lists[k]);
    fclose(f);
    return rc;
}
