/* nn_internal.h -- accessors shared between the optimizer and EMA modules. */
#ifndef NN_INTERNAL_H
#define NN_INTERNAL_H

#include "nn_modules.h"

int nn_ema_count(const EMA* ema);
float nn_ema_decay(const EMA* ema);
float* nn_ema_shadow(const EMA* ema, int i);

#endif /* NN_INTERNAL_H */
