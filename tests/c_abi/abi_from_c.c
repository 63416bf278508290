/* The C-ABI used from plain C11, as a Swift module map over the header
 * would import it: the header compiles as C, and the host-side entry points
 * (argument and geometry checks, host tables) behave as documented.  No
 * entry point here reaches a GPU call. */
#include <stdio.h>
#include <string.h>

#include "minirun_hip.h"

static int failures = 0;
#define EXPECT(cond)                                                   \
    do {                                                               \
        if (!(cond)) {                                                 \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                                \
        }                                                              \
    } while (0)

int main(void) {
    EXPECT(strncmp(mr_version(), "minirun-hip", 11) == 0);

    /* AffineWeights validation: a valid q_a operand, then a wrong packed dtype */
    int64_t ps[2] = {1536, 896}, ss[2] = {1536, 112}, experts = -1, out_f = 0, in_f = 0;
    EXPECT(mr_affine_validate(MR_U32, 2, ps, MR_BF16, 2, ss, MR_BF16, 2, ss, 64, 4, &experts, &out_f, &in_f) == MR_OK);
    EXPECT(experts == 0 && out_f == 1536 && in_f == 7168);
    EXPECT(mr_affine_validate(MR_F32, 2, ps, MR_BF16, 2, ss, MR_BF16, 2, ss, 64, 4, &experts, &out_f, &in_f) ==
           MR_INVALID_DTYPE);
    EXPECT(strstr(mr_get_last_error(), "uint32") != NULL);

    /* lightning-index selection geometry and the scores' geometry check */
    int32_t selected = -1;
    EXPECT(mr_topk_geometry(1, 32768, 2048, 4, 131071, 0, &selected) == MR_OK && selected == 2048);
    EXPECT(mr_topk_geometry(2, 4, 2, 1, 3, 0, &selected) == MR_INVALID_SHAPE);
    EXPECT(mr_indexer_scores(NULL, MR_BF16, 1, 64, 128, 8192, 128, NULL, MR_BF16, 16, 64, 64, NULL, MR_F32, 1, 64, 64,
                             NULL, 16, NULL) == MR_INVALID_SHAPE);
    EXPECT(strstr(mr_get_last_error(), "incompatible geometry") != NULL);
    EXPECT(mr_indexer_scores(NULL, MR_BF16, 1, 64, 128, 8192, 128, NULL, MR_BF16, 0, 128, 128, NULL, MR_F32, 1, 64,
                             64, NULL, 0, NULL) == MR_OK); /* no keys: nothing to do */

    /* window index table: 3 tokens from position 0, window 4 */
    int32_t tab[16], rows = 0, cols = 0;
    EXPECT(mr_attention_indices_window(4, 3, 0, tab, &rows, &cols) == MR_OK);
    EXPECT(rows == 3 && cols == 3);
    EXPECT(tab[0] == 0 && tab[1] == -1 && tab[3] == 0 && tab[4] == 1 && tab[8] == 2);

    /* rotary frequencies: f_0 = 1 */
    double freqs[32];
    EXPECT(mr_rope_frequencies(64, 0, 10000.0, 1.0, 32.0, 1.0, freqs) == MR_OK);
    EXPECT(freqs[0] == 1.0 && freqs[1] < 1.0);

    /* decode arguments are checked before any device work */
    mr_mla_decode_args a;
    memset(&a, 0, sizeof a);
    a.batch = 1;
    a.heads = 16;
    a.n_ctx = 512;
    a.kv_rank = 4096; /* beyond every kernel's widths */
    a.rope_dim = 64;
    a.scale = 0.07f;
    EXPECT(mr_mla_decode(&a, NULL) == MR_INVALID_SHAPE);
    a.kv_rank = 256; /* the any-width kernel's: on to the pointer checks */
    EXPECT(mr_mla_decode(&a, NULL) == MR_INVALID_ARGUMENT);
    EXPECT(mr_mla_decode(NULL, NULL) == MR_INVALID_ARGUMENT);

    /* the prefill block: workspace geometry, then shape and pointer checks */
    mr_mla_prefill_block_args pb;
    memset(&pb, 0, sizeof pb);
    EXPECT(mr_mla_prefill_block_workspace_size(NULL) == 0);
    EXPECT(mr_mla_prefill_block_workspace_size(&pb) == 0); /* no tokens */
    pb.tokens = 64;
    pb.hidden = 256;
    pb.q_lora_rank = 64;
    pb.heads = 4;
    pb.qk_nope_dim = 32;
    pb.qk_rope_dim = 16;
    pb.v_head_dim = 32;
    pb.kv_rank = 64;
    pb.capacity = 64;
    EXPECT(mr_mla_prefill_block_workspace_size(&pb) > 0);
    pb.kv_rank = -64; /* a width the call rejects: no size */
    EXPECT(mr_mla_prefill_block_workspace_size(&pb) == 0);
    pb.kv_rank = 64;
    EXPECT(mr_mla_prefill_block(&pb, NULL) == MR_INVALID_ARGUMENT); /* no pointers */
    EXPECT(strstr(mr_get_last_error(), "NULL") != NULL);
    pb.capacity = 63; /* rows 0 .. 63 do not fit */
    EXPECT(mr_mla_prefill_block(&pb, NULL) == MR_INVALID_SHAPE);
    pb.capacity = 64;
    pb.qk_rope_dim = 15;
    EXPECT(mr_mla_prefill_block(&pb, NULL) == MR_INVALID_SHAPE);
    EXPECT(mr_mla_prefill_block(NULL, NULL) == MR_INVALID_ARGUMENT);

    if (failures) return 1;
    printf("abi_from_c: ok\n");
    return 0;
}
