/*
 * CPU oracle of the ragged packer -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates, for a flat stream of tokenizer words, what the reference does
 * per batch in UCITokenizer.pad_and_collate (src/modeling/data.py:281-337):
 *   - keep the FIRST max_len words of each game (data.py:290);
 *   - input id = word & 0x3FFF (data.py:320);
 *   - position id = (cumsum(attention_mask) - 1).clamp(0) (data.py:327),
 *     which on the real (non-pad) tokens of a game is 0..n-1 as long as no
 *     PAD id occurs inside the game (the tokenizer never writes one there;
 *     such a game is flagged with status bit 8);
 * and lays the result out ragged instead of right-padded:
 *   cu_seqlens[B+1]   exclusive scan of n_i = min(len_i, max_len)
 *   ids[T], pos[T], seq_of[T]   per token
 *   last_idx[B] = cu_seqlens[i+1] - 1   (the row whose logits the callers
 *                 read as [:, -1], decode.py:204,366)
 *   blk_off[B+1]      exclusive scan of ceil(n_i / block)
 *   block_table[B][max_blocks]  block ids first_block + blk_off[i] + j, -1 past the end
 *   slot[T] = block_table[s][p / block] * block + p % block
 * Returns a status bitmask with the engine's meaning: 0 ok, 1 an empty
 * game, 4 a block table too small (nothing written for that game's tokens
 * beyond the table), 8 the id pad_id inside a game.
 * Built by oracle/Makefile into oracle/_build/liboracle.so.
 */
#include <stdint.h>

int oracle_pack(const uint32_t *words, const int32_t *lens, int B, int max_len,
                int block, int first_block, int max_blocks, int pad_id,
                int32_t *cu_seqlens, int32_t *ids, int32_t *pos, int32_t *seq_of,
                int32_t *last_idx, int32_t *blk_off, int32_t *block_table,
                int32_t *slot) {
  int64_t in_off = 0;
  int32_t t = 0, nb_total = 0;
  int status = 0;
  cu_seqlens[0] = 0;
  blk_off[0] = 0;
  for (int s = 0; s < B; ++s) {
    int n = lens[s] > 0 ? lens[s] : 0;
    if (n == 0) status |= 1;
    if (n > max_len) n = max_len;
    int nb = (n + block - 1) / block;
    if (nb > max_blocks) status |= 4;
    for (int j = 0; j < max_blocks; ++j)
      block_table[(int64_t)s * max_blocks + j] = j < nb ? first_block + nb_total + j : -1;
    for (int j = 0; j < n; ++j) {
      uint32_t w = words[in_off + j];
      ids[t + j] = (int32_t)(w & 0x3FFFu);
      if (ids[t + j] == pad_id) status |= 8;
      pos[t + j] = j;
      seq_of[t + j] = s;
      slot[t + j] = (first_block + nb_total + j / block) * block + j % block;
    }
    t += n;
    nb_total += nb;
    in_off += lens[s] > 0 ? lens[s] : 0;
    cu_seqlens[s + 1] = t;
    last_idx[s] = t - 1;
    blk_off[s + 1] = nb_total;
  }
  return status;
}
