/*
 * mha_decode_int.h — params of the MHA_Decode operator.
 *
 * Layout-identical to src/operator/nn/mha_decode_int.h:6-15 of the reference
 * (seven int64 fields and one float, 64 bytes), which graph_update_cache_len relies on.
 *
 * Extension (absent in the reference, opt-in only): cache_len < 0 selects ragged mode.
 * The op then reads per-sequence cache lengths from one extra input slot (index 11),
 * an int32 device array of B entries; sequence b attends positions 0..len[b] after
 * appending its new token at position len[b].  cache_len == -2 is the same with the
 * caller's guarantee that all B lengths are equal (a uniform length kept on the device,
 * as graph_execute does so that a recorded step replays at every length): the op then
 * plans and runs as for a uniform length, over max_seq positions.  cache_len == -3 is
 * -2 for the full op whose last kernel also adds one to each of the B lengths after the
 * step (a recorded decode step then advances its own position; the attention-only entry
 * rejects -3).  Device-held lengths cannot be checked on the host: a length >= max_seq
 * appends nothing and attends max_seq positions, a negative one appends nothing and
 * attends position 0 only; Q is projected either way (the RoPE variants then leave it
 * unrotated, having no angle for that position).
 */
#ifndef CF_MHA_DECODE_INT_H_
#define CF_MHA_DECODE_INT_H_

#include <stdint.h>

typedef struct {
    int64_t batch_size;   /* B */
    int64_t hidden_size;  /* D */
    int64_t num_heads;    /* H_q — query heads */
    int64_t num_kv_heads; /* H_kv — key/value heads (GQA: H_kv < H_q); <= 0 means H_q */
    int64_t head_dim;     /* d */
    float   scale;        /* usually 1/sqrt(d) */
    int64_t cache_len;    /* position of the new token; < 0 = ragged (lengths in slot 11) */
    int64_t max_seq;      /* cache capacity in positions */
} mha_decode_params_t;

#define MHA_DECODE_NUM_INPUTS   11
#define MHA_DECODE_NUM_OUTPUTS  3
#define MHA_DECODE_SLOT_SEQLENS 11
#define MHA_DECODE_CACHE_LEN_DEVICE_UNIFORM (-2)
#define MHA_DECODE_CACHE_LEN_DEVICE_ADVANCE (-3)

#endif /* CF_MHA_DECODE_INT_H_ */
