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

/* Payloads are read through one host staging buffer of at most this many
   floats; a chunk may span several tensors of the list. */
#define CK_STAGE_FLOATS ((size_t)1 << 22)

/* One list in the layout write_list produces.  The header is validated in
   file order before any payload is read: the count (-3 when it differs from
   the model's), then the sizes, where the first entry that differs from the
   model's tensor gives -4 even if the file also ends early, and a file that
   ends inside the header or the payloads gives -2.  Payloads are contiguous
   in the file, so they stream in chunks and are uploaded tensor by tensor. */
static int read_list(FILE* f, ParamList* pl)
{
    int count = 0;
    if (ck_read(&count, sizeof count, 1, f)) return -2;
    if (count != pl->count) {
        fprintf(stderr, "checkpoint: the file lists %d tensors where the model has %d\n", count, pl->count);
        return -3;
    }
    int* sizes = (int*)malloc((size_t)(count > 0 ? count : 1) * sizeof(int));
    const size_t got = fread(sizes, sizeof(int), (size_t)count, f);
    size_t total = 0;
    for (size_t i = 0; i < got; ++i) {
        if (sizes[i] != pl->items[i].size) {
            fprintf(stderr, "checkpoint: tensor %zu holds %d floats in the file and %d in the model\n", i,
                sizes[i], pl->items[i].size);
            free(sizes);
            return -4;
        }
        total += (size_t)sizes[i];
    }
    free(sizes);
    if (got != (size_t)count) return -2;

    const size_t cap = total < CK_STAGE_FLOATS ? total : CK_STAGE_FLOATS;
    float* stage = (float*)malloc((cap ? cap : 1) * sizeof(float));
    int t = 0;         /* tensor being filled */
    size_t done = 0;   /* floats of tensor t already uploaded */
    size_t left = total;
    int rc = 0;
    while (left && !rc) {
        const size_t chunk = left < cap ? left : cap;
        if (ck_read(stage, sizeof(float), chunk, f)) {
            rc = -2;
            break;
        }
        left -= chunk;
        for (size_t at = 0; at < chunk;) {
            while ((size_t)pl->items[t].size == done) { /* skip finished (and empty) tensors */
                ++t;
                done = 0;
            }
            const size_t want = (size_t)pl->items[t].size - done;
            const size_t take = chunk - at < want ? chunk - at : want;
            NN_HIP_CHECK(hipMemcpy(pl->items[t].param + done, stage + at, take * sizeof(float),
                hipMemcpyHostToDevice));
            done += take;
            at += take;
        }
    }
    free(stage);
    return rc;
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
