/* Host chess rules for the search (liballie_chess.so, allie_amd/csrc/chess.cpp).
 *
 * Replaces what the reference takes from python-chess on its search path:
 *   - Game.board: chess.Board() replayed with push_uci (src/modeling/data.py:51-56)
 *     -> allie_chess_start, allie_chess_push_uci (one move on a parent position);
 *   - Game.legal_moves: [m.uci() for m in board.legal_moves] (data.py:58-61)
 *     -> allie_chess_legal_uci, in python-chess's generation order;
 *   - board.outcome() in MCTS.evaluate_node / AdaptiveMCTS.evaluate_root
 *     (src/evaluation/decode.py:345-353, 518-530) -> allie_chess_outcome.
 * Positions are immutable heap objects owned by the caller (allie_chess_free).
 * No GPU code; thread-safe for distinct or shared read-only positions. */
#ifndef ALLIE_CHESS_H
#define ALLIE_CHESS_H

#ifdef __cplusplus
extern "C" {
#endif

void* allie_chess_start(void);                 /* the initial position, or NULL (no memory) */
void* allie_chess_from_fen(const char* fen);   /* a FEN position without history, or NULL */
void allie_chess_free(void* pos);
/* the position after a legal UCI move ("e2e4", "e7e8q"), or NULL when the
 * move is malformed or illegal (python-chess push_uci raises there) */
void* allie_chess_push_uci(const void* pos, const char* uci);
/* legal moves as space-separated UCI, NUL-terminated; returns their count,
 * or -(bytes needed) when cap is too small (2048 always suffices) */
int allie_chess_legal_uci(const void* pos, char* out, int cap);
/* 0 while the game goes on, else termination * 4 + winner, winner 0 draw,
 * 1 white, 2 black; terminations 1 checkmate, 2 insufficient material,
 * 3 stalemate, 4 seventy-five moves, 5 fivefold repetition (the order of
 * python-chess outcome(claim_draw=False)) */
int allie_chess_outcome(const void* pos);
int allie_chess_is_check(const void* pos);
int allie_chess_white_to_move(const void* pos);
long long allie_chess_perft(const void* pos, int depth);

#ifdef __cplusplus
}
#endif
#endif
