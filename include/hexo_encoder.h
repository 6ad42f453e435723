/*
 * hexo_encoder.h — C ABI of the native Hexo rules subset and MantisNet
 * position encoder (host code, libhexo_encoder.so).
 *
 * This library replaces the Rust/PyO3 pieces the MantisNet leaf-evaluation
 * path reaches for its inputs.  Every entry point takes plain pointers and
 * sizes, returns 0 on success or a nonzero status, and writes a readable
 * message into `err` (when `err_len` > 0) on failure.  Nothing here touches a
 * GPU.  All entry points are re-entrant; a HexoBatch is immutable after build.
 */
#ifndef HEXO_ENCODER_H
#define HEXO_ENCODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define HEXO_OK 0
#define HEXO_E_ARG 1      /* malformed arguments (sizes, pointers, ranges) */
#define HEXO_E_ILLEGAL 2  /* an illegal move in a replayed game */
#define HEXO_E_TERMINAL 3 /* a terminal position was handed to the builder */
#define HEXO_E_LIMIT 4    /* a representation limit was exceeded */
#define HEXO_E_INTERNAL 5 /* an encoder invariant failed */
#define HEXO_E_WIRE 6     /* a wire item failed validation */

/* Field dtypes reported by hexo_batch_field. */
#define HEXO_I64 1
#define HEXO_I32 2
#define HEXO_BOOL 3
#define HEXO_F32 4

typedef struct HexoBatch HexoBatch;

/* Version of the batch representation this library emits (the value of
 * MODEL_REPR_VERSION it restates; python/hexo-py/src/lib.rs:19-30). */
int32_t hexo_repr_version(void);

/*
 * Replay the first ts[i] placements of each game and collate the built
 * graphs into one batch.  Replaces hexo_py.build_batch_prefixes
 * (python/hexo-py/src/lib.rs:278-310 -> encoder.rs:1648-1671) and, with
 * ts[i] = full game length, hexo_py.build_batch over replayed positions
 * (lib.rs:266-276 -> encoder.rs:1642-1646).
 *   moves_qr      (total, 2) int16 placements, games concatenated
 *   move_offsets  (n_games + 1) int64 CSR offsets into moves_qr
 *   ts            (n_games) int64 prefix length per game
 *   n_threads     worker threads (<= 0: hardware concurrency)
 * On success *out owns the batch; release it with hexo_batch_free.
 */
int32_t hexo_build_batch_prefixes(int64_t n_games, const int16_t* moves_qr,
                                  const int64_t* move_offsets, const int64_t* ts,
                                  int32_t n_threads, HexoBatch** out, char* err,
                                  int64_t err_len);

/*
 * The rules state after replaying `n_moves` placements, terminal positions
 * included (hexo_py.Position, python/hexo-py/src/lib.rs:40-199): the legal
 * placements in canonical order (none once terminal; up to `cap` pairs
 * written, the count in *n_legal), the side to move (frozen at the winner
 * once terminal), the placements it has left this turn, the winner (-1 while
 * the game runs) and the stone count.  An illegal placement, or one after
 * the game ended, fails with HEXO_E_ILLEGAL.
 */
int32_t hexo_position_state(int64_t n_moves, const int16_t* moves_qr, int64_t cap, int16_t* legal_qr,
                            int64_t* n_legal, int32_t* mover, int32_t* moves_remaining, int32_t* winner,
                            int64_t* n_stones, char* err, int64_t err_len);

/*
 * One live position as the versioned worker-to-batcher wire item
 * (encoder.rs:539-621: magic "MANTIS\0\1", MODEL_REPR_VERSION, the side's
 * remaining placements, seven u32 counts, then the position's graph arrays,
 * little-endian).  Replays n_moves placements, builds, and writes the item
 * into `out` when `cap` holds it; *len always receives the item's length
 * (call with cap = 0 to size the buffer).  Replaces encoder::encode_position
 * (used by seam.rs:15).
 */
int32_t hexo_encode_position(int64_t n_moves, const int16_t* moves_qr, uint8_t* out, int64_t cap,
                             int64_t* len, char* err, int64_t err_len);

/*
 * Validate and collate n_items wire items (item i = bytes[item_offsets[i] ..
 * item_offsets[i+1])) into one batch, as hexo_build_batch_prefixes does for
 * replayed games.  Every check of encoder.rs:666-941 runs before collation
 * (magic, version, remaining placements, reserved bytes, counts capped at the
 * item length, exact length, every feature's domain and index bound, the
 * action rows against the decoder incidences, the tactical range and its
 * nonempty column); the first failure returns HEXO_E_WIRE with the item and
 * the reason in `err`.  Replaces encoder::decode_batch (encoder.rs:1632-1639,
 * used by seam.rs:83).
 */
int32_t hexo_decode_batch(int64_t n_items, const uint8_t* bytes, const int64_t* item_offsets,
                          int32_t n_threads, HexoBatch** out, char* err, int64_t err_len);

/* The batch's scalar sizes (builder.py:666-700: n_pos, max_t, max_w, n_cells). */
int32_t hexo_batch_scalars(const HexoBatch* batch, int64_t* n_pos, int64_t* max_t,
                           int64_t* max_w, int64_t* n_cells);

/*
 * Borrow one collated field by its Batch name (builder.py:666-752 and the
 * dict keys of lib.rs:191-258, plus the seven relay_* views).  Returns the
 * dtype code (HEXO_I64/I32/BOOL/F32) and the element count; 0 if the name is
 * unknown.  The pointer stays valid until hexo_batch_free.
 */
int32_t hexo_batch_field(const HexoBatch* batch, const char* name, const void** data,
                         int64_t* numel);

void hexo_batch_free(HexoBatch* batch);

/*
 * The seven relay CSR views of a decoder incidence (relay.py:48-94, run by
 * builder.batch_from_arrays for every batch, builder.py:764-811).
 *   inputs  dec_cell/dec_window/dec_class (e) int64
 *   outputs cell_ptr (n_covered + 1; caller passes capacity e + 1 and gets
 *           the count in *n_covered), window/class/wcell/ccell (e),
 *           win_ptr (n_windows + 1), cls_ptr (n_classes + 1)
 */
int32_t hexo_relay_tables(int64_t e, const int64_t* dec_cell, const int64_t* dec_window,
                          const int64_t* dec_class, int64_t n_windows, int64_t n_classes,
                          int64_t* cell_ptr, int64_t* n_covered, int64_t* window,
                          int64_t* cls, int64_t* win_ptr, int64_t* wcell,
                          int64_t* cls_ptr, int64_t* ccell, char* err, int64_t err_len);

/*
 * Legal placements after replaying `n_moves` placements, in canonical
 * ascending (q, r) order (hexo_py.Position.legal_moves, lib.rs:74-84).
 * Writes up to `cap` (q, r) pairs and the count to *n_legal; also the side
 * to move and the placements left this turn (lib.rs:145-153).
 */
int32_t hexo_legal_moves(int64_t n_moves, const int16_t* moves_qr, int64_t cap,
                         int16_t* legal_qr, int64_t* n_legal, int32_t* mover,
                         int32_t* moves_remaining, char* err, int64_t err_len);

/*
 * Seeded random legal play (the synthetic-position generator of the
 * benchmark configurations; it has no counterpart in the reference):
 * P0 opens at the origin, then every placement is drawn as
 * floor(u[ply] * n) among the n canonical-order legal cells that do not
 * complete six in a row for the mover.  Writes n_stones placements.
 */
int32_t hexo_random_game(int64_t n_stones, const double* u, int16_t* moves_qr,
                         char* err, int64_t err_len);

/*
 * Vocabulary tables (builder.py:88-229, encoder.rs:140-302, 55-107):
 * rank (729), dec/occ/post1 (729*6), orbit (25*25 indexed [dq+12][dr+12]),
 * pattern_counts (377*1458 float32).  Any pointer may be NULL.
 */
int32_t hexo_tables(int32_t* rank, int32_t* dec, int32_t* occ, int32_t* post1,
                    int32_t* orbit, float* pattern_counts);

#ifdef __cplusplus
}
#endif

#endif
