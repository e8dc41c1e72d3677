/*
 * Shared by oracle/sc_oracle.c and oracle/sc_fastgemm.c (test
 * infrastructure only): the config mirror, status codes and the two config
 * helpers sc_oracle.c defines.
 */
#ifndef SC_ORACLE_CFG_H
#define SC_ORACLE_CFG_H

#include <stdint.h>

#define ORC_INVALID_NEIGHBOR (-1) /* crates/burn_flex_gmm/src/lib.rs:3 */

/* Mirror of SparseSubmConvConfig, crates/burn_flex_gmm/src/lib.rs:5-17. */
typedef struct orc_cfg {
    int64_t in_channels;
    int64_t out_channels;
    int64_t kernel_d;
    int64_t kernel_h;
    int64_t kernel_w;
    int64_t in_channels_per_group;
    int64_t out_channels_per_group;
    int64_t groups;
    int32_t axis_order[3];
    int32_t axis_sign[3];
} orc_cfg;

enum {
    ORC_OK = 0,
    ORC_ERR_CONFIG = 1,
    ORC_ERR_SHAPE = 2,
    ORC_ERR_INDEX = 3,
    ORC_ERR_ALLOC = 4,
};

int orc_validate_config(const orc_cfg *c);
int64_t orc_kernel_rows(const orc_cfg *c);

#endif
