/* gpt2_config.h -- GPT-2-124M dimensions.  Replaces model/config.h:11-42 (same macro names and
 * values, so host code written against the reference's config.h compiles unchanged). Plain C. */
#ifndef GPT2_CONFIG_H
#define GPT2_CONFIG_H

#define GPT2_N_LAYER 12
#define GPT2_N_HEAD 12
#define GPT2_N_EMBD 768
#define GPT2_VOCAB 50257
#define GPT2_N_CTX 1024
#define GPT2_HEAD_DIM (GPT2_N_EMBD / GPT2_N_HEAD) /* 64 */
#define GPT2_FFN_DIM (4 * GPT2_N_EMBD)            /* 3072 */
#define GPT2_QKV_DIM (3 * GPT2_N_EMBD)            /* 2304 */
#define GPT2_LN_EPS 1e-5f

/* 50257*768 + 1024*768 + 12*(2*768 + 2304*768 + 2304 + 768*768 + 768 + 2*768 + 3072*768 + 3072
 *  + 768*3072 + 768) + 2*768 */
#define GPT2_TOTAL_PARAMS 124439808L

#endif
