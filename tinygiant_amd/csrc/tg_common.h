/*
 * tg_common.h -- constants shared by the host and device sides of
 * libtinygiant_hip.  Format and activation codes are the reference's
 * (csrc/libtinygiant.c:594 and :1248; tinygiant/engine.py:20-22).
 */
#ifndef TG_COMMON_H
#define TG_COMMON_H

enum { TG_FMT_Q4K = 0, TG_FMT_F16 = 1, TG_FMT_Q6K = 2, TG_FMT_MXFP4 = 3, TG_FMT_Q80 = 4 };
enum { TG_ACT_SILU = 0, TG_ACT_GPTOSS = 1 };

#define TG_QK 256            /* values per q8 activation block */
#define TG_Q8_NB(n) (((n) + TG_QK - 1) / TG_QK)

#endif
