// Host chess rules for the search: legal moves in python-chess's generation
// order, game-over detection and perft, behind a C ABI (include/allie_chess.h).
//
// The reference gets these from python-chess: Game.board replays the game
// with push_uci, Game.legal_moves lists board.legal_moves as UCI
// (src/modeling/data.py:51-61), and MCTS asks board.outcome()
// (src/evaluation/decode.py:345-353).  python-chess is absent from the image;
// oracle/movegen.py restates the rules in Python and fixes the order this
// file follows:
//   not in check: pieces other than pawns by from-square descending (a1 = 0),
//   targets descending; castling, king side first; pawn captures by
//   from-square descending, targets descending; single pushes, then double
//   pushes, by target descending; en passant by capturer descending;
//   promotions q, r, b, n.
//   in check: king moves (targets descending); against one checker the
//   other pieces' moves (order above) that capture it or block its line;
//   then an en passant capture of a checking pawn.
// Game over: checkmate, insufficient material, stalemate, 150 half-moves,
// fivefold repetition (keys: placement, side, castling rights, and the
// en passant square only when a legal en passant capture exists).
//
// A position is an immutable node: push returns a new one.  Repetition keys
// are kept from the last irreversible move on (a capture or pawn move makes
// every earlier position unreachable), so a node holds at most 151 keys.

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

namespace {

enum : uint8_t { EMPTY = 0, PAWN = 1, KNIGHT = 2, BISHOP = 3, ROOK = 4, QUEEN = 5, KING = 6, BLACK = 8 };
enum : uint8_t { CW_K = 1, CW_Q = 2, CB_K = 4, CB_Q = 8 };

struct Move {
  uint8_t from, to, promo;  // promo: 0 or QUEEN/ROOK/BISHOP/KNIGHT
};

// ------------------------------------------------------------------ tables
struct Tables {
  // step targets in the Python generator's delta order
  uint8_t knight[64][8], n_knight[64];
  uint8_t king[64][8], n_king[64];
  // rays: orthogonal (E, W, N, S) then diagonal (NE, SE, NW, SW)
  uint8_t ray[64][8][7], n_ray[64][8];
  uint64_t z_piece[16][64], z_side, z_castle[16], z_ep[64];
  Tables() {
    const int kd[8][2] = {{1, 2}, {2, 1}, {2, -1}, {1, -2}, {-1, -2}, {-2, -1}, {-2, 1}, {-1, 2}};
    const int gd[8][2] = {{1, 0}, {1, 1}, {0, 1}, {-1, 1}, {-1, 0}, {-1, -1}, {0, -1}, {1, -1}};
    const int rd[8][2] = {{1, 0}, {-1, 0}, {0, 1}, {0, -1}, {1, 1}, {1, -1}, {-1, 1}, {-1, -1}};
    for (int s = 0; s < 64; ++s) {
      const int f = s & 7, r = s >> 3;
      n_knight[s] = n_king[s] = 0;
      for (auto& d : kd)
        if (f + d[0] >= 0 && f + d[0] < 8 && r + d[1] >= 0 && r + d[1] < 8)
          knight[s][n_knight[s]++] = (uint8_t)((r + d[1]) * 8 + f + d[0]);
      for (auto& d : gd)
        if (f + d[0] >= 0 && f + d[0] < 8 && r + d[1] >= 0 && r + d[1] < 8)
          king[s][n_king[s]++] = (uint8_t)((r + d[1]) * 8 + f + d[0]);
      for (int k = 0; k < 8; ++k) {
        n_ray[s][k] = 0;
        int nf = f + rd[k][0], nr = r + rd[k][1];
        while (nf >= 0 && nf < 8 && nr >= 0 && nr < 8) {
          ray[s][k][n_ray[s][k]++] = (uint8_t)(nr * 8 + nf);
          nf += rd[k][0];
          nr += rd[k][1];
        }
      }
    }
    uint64_t x = 0x9E3779B97F4A7C15ull;  // splitmix64 stream
    auto next = [&]() {
      x += 0x9E3779B97F4A7C15ull;
      uint64_t z = x;
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      return z ^ (z >> 31);
    };
    for (auto& row : z_piece)
      for (auto& v : row) v = next();
    z_side = next();
    for (auto& v : z_castle) v = next();
    for (auto& v : z_ep) v = next();
  }
};
const Tables T;

// ------------------------------------------------------------------- board
struct Board {
  uint8_t sq[64];
  bool white;
  uint8_t castling;
  int8_t ep;  // -1: none
  int halfmove;
  std::vector<uint64_t> keys;  // since the last irreversible move, current last

  bool ours(uint8_t p) const { return p != EMPTY && ((p & BLACK) == 0) == white; }

  bool attacked_by(int s, bool by_white) const {
    const uint8_t c = by_white ? 0 : BLACK;
    for (int i = 0; i < T.n_knight[s]; ++i)
      if (sq[T.knight[s][i]] == (KNIGHT | c)) return true;
    for (int i = 0; i < T.n_king[s]; ++i)
      if (sq[T.king[s][i]] == (KING | c)) return true;
    for (int k = 0; k < 8; ++k) {
      const uint8_t a = k < 4 ? ROOK : BISHOP;
      for (int i = 0; i < T.n_ray[s][k]; ++i) {
        const uint8_t p = sq[T.ray[s][k][i]];
        if (p != EMPTY) {
          if (p == (a | c) || p == (QUEEN | c)) return true;
          break;
        }
      }
    }
    const int f = s & 7, r = s >> 3, pr = by_white ? r - 1 : r + 1;
    if (pr >= 0 && pr < 8)
      for (int df = -1; df <= 1; df += 2)
        if (f + df >= 0 && f + df < 8 && sq[pr * 8 + f + df] == (PAWN | c)) return true;
    return false;
  }

  int king_square(bool w) const {
    const uint8_t k = KING | (w ? 0 : BLACK);
    for (int s = 0; s < 64; ++s)
      if (sq[s] == k) return s;
    return -1;
  }

  bool is_check() const {
    const int k = king_square(white);
    return k >= 0 && attacked_by(k, !white);
  }

  int checkers(int* out) const {
    const int k = king_square(white);
    const uint8_t c = white ? BLACK : 0;
    int n = 0;
    for (int i = 0; i < T.n_knight[k]; ++i)
      if (sq[T.knight[k][i]] == (KNIGHT | c)) out[n++] = T.knight[k][i];
    for (int k2 = 0; k2 < 8; ++k2) {
      const uint8_t a = k2 < 4 ? ROOK : BISHOP;
      for (int i = 0; i < T.n_ray[k][k2]; ++i) {
        const int t = T.ray[k][k2][i];
        const uint8_t p = sq[t];
        if (p != EMPTY) {
          if (p == (a | c) || p == (QUEEN | c)) out[n++] = t;
          break;
        }
      }
    }
    const int f = k & 7, r = k >> 3, pr = white ? r + 1 : r - 1;
    if (pr >= 0 && pr < 8)
      for (int df = -1; df <= 1; df += 2)
        if (f + df >= 0 && f + df < 8 && sq[pr * 8 + f + df] == (PAWN | c)) out[n++] = pr * 8 + f + df;
    return n;
  }

  // targets of a non-pawn piece, unsorted (caller sorts descending)
  int piece_targets(int s, int t, uint8_t* out) const {
    int n = 0;
    if (t == KNIGHT) {
      for (int i = 0; i < T.n_knight[s]; ++i) out[n++] = T.knight[s][i];
      return n;
    }
    if (t == KING) {
      for (int i = 0; i < T.n_king[s]; ++i) out[n++] = T.king[s][i];
      return n;
    }
    const int k0 = t == BISHOP ? 4 : 0, k1 = t == ROOK ? 4 : 8;
    for (int k = k0; k < k1; ++k)
      for (int i = 0; i < T.n_ray[s][k]; ++i) {
        const int u = T.ray[s][k][i];
        out[n++] = (uint8_t)u;
        if (sq[u] != EMPTY) break;
      }
    return n;
  }

  static void sort_desc(uint8_t* a, int n) {
    for (int i = 1; i < n; ++i) {
      const uint8_t v = a[i];
      int j = i - 1;
      while (j >= 0 && a[j] < v) {
        a[j + 1] = a[j];
        --j;
      }
      a[j + 1] = v;
    }
  }

  void add_pawn(std::vector<Move>& m, int s, int u) const {
    const int last = white ? 7 : 0;
    if ((u >> 3) == last) {
      const uint8_t pr[4] = {QUEEN, ROOK, BISHOP, KNIGHT};
      for (uint8_t p : pr) m.push_back({(uint8_t)s, (uint8_t)u, p});
    } else {
      m.push_back({(uint8_t)s, (uint8_t)u, 0});
    }
  }

  void ep_moves(std::vector<Move>& m) const {
    if (ep < 0) return;
    const uint8_t pawn = PAWN | (white ? 0 : BLACK);
    const int e = ep, f = e & 7, rf = white ? (e >> 3) - 1 : (e >> 3) + 1;
    for (int df = 1; df >= -1; df -= 2)  // capturer squares descending
      if (f + df >= 0 && f + df < 8 && sq[rf * 8 + f + df] == pawn) m.push_back({(uint8_t)(rf * 8 + f + df), (uint8_t)e, 0});
  }

  void castling_moves(std::vector<Move>& m) const {
    const int rank = white ? 0 : 56;
    const uint8_t king = KING | (white ? 0 : BLACK), rook = ROOK | (white ? 0 : BLACK);
    if (sq[rank + 4] != king) return;
    struct Side {
      uint8_t right, rook_sq, ne, empty[3], safe[3], to;
    };
    const Side sides[2] = {
        {(uint8_t)(white ? CW_K : CB_K), (uint8_t)(rank + 7), 2, {5, 6, 0}, {4, 5, 6}, (uint8_t)(rank + 6)},
        {(uint8_t)(white ? CW_Q : CB_Q), (uint8_t)(rank + 0), 3, {1, 2, 3}, {4, 3, 2}, (uint8_t)(rank + 2)},
    };
    for (const Side& sd : sides) {
      if (!(castling & sd.right) || sq[sd.rook_sq] != rook) continue;
      bool ok = true;
      for (int i = 0; i < sd.ne && ok; ++i) ok = sq[rank + sd.empty[i]] == EMPTY;
      for (int i = 0; i < 3 && ok; ++i) ok = !attacked_by(rank + sd.safe[i], !white);
      if (ok) m.push_back({(uint8_t)(rank + 4), sd.to, 0});
    }
  }

  // pseudo-legal moves in the generation order; to_ok: 64-bit target mask
  // (all ones: unrestricted)
  void pseudo(std::vector<Move>& m, uint64_t to_ok, bool kings) const {
    const bool any = to_ok == ~0ull;
    uint8_t tg[32];
    for (int s = 63; s >= 0; --s) {
      const uint8_t p = sq[s];
      if (p == EMPTY || !ours(p) || (p & 7) == PAWN) continue;
      if ((p & 7) == KING && !kings) continue;
      const int n = piece_targets(s, p & 7, tg);
      sort_desc(tg, n);
      for (int i = 0; i < n; ++i)
        if (!ours(sq[tg[i]]) && ((to_ok >> tg[i]) & 1)) m.push_back({(uint8_t)s, tg[i], 0});
    }
    if (kings && any) castling_moves(m);
    const uint8_t pawn = PAWN | (white ? 0 : BLACK);
    const int fwd = white ? 8 : -8;
    for (int s = 63; s >= 0; --s) {  // captures
      if (sq[s] != pawn) continue;
      const int f = s & 7;
      for (int df = 1; df >= -1; df -= 2) {
        if (f + df < 0 || f + df >= 8) continue;
        const int u = s + fwd + df;
        if (u < 0 || u >= 64) continue;  // a pawn on its last rank (possible only from a FEN)
        if (sq[u] != EMPTY && !ours(sq[u]) && ((to_ok >> u) & 1)) add_pawn(m, s, u);
      }
    }
    // single pushes by target descending: for white targets = from + 8, the
    // from-squares in descending order give descending targets (black too)
    for (int s = 63; s >= 0; --s) {
      if (sq[s] != pawn) continue;
      const int u = s + fwd;
      if (u < 0 || u >= 64) continue;
      if (sq[u] == EMPTY && ((to_ok >> u) & 1)) add_pawn(m, s, u);
    }
    const int start = white ? 1 : 6;
    for (int s = 63; s >= 0; --s) {
      if (sq[s] != pawn || (s >> 3) != start) continue;
      const int u = s + 2 * fwd;
      if (sq[s + fwd] == EMPTY && sq[u] == EMPTY && ((to_ok >> u) & 1)) m.push_back({(uint8_t)s, (uint8_t)u, 0});
    }
    if (ep >= 0 && ((to_ok >> ep) & 1)) ep_moves(m);
  }

  void make(const Move& mv, Board& b) const {
    std::memcpy(b.sq, sq, 64);
    const int s = mv.from, u = mv.to;
    const uint8_t p = sq[s], t = p & 7;
    bool cap = sq[u] != EMPTY;
    b.sq[u] = mv.promo ? (uint8_t)(mv.promo | (p & BLACK)) : p;
    b.sq[s] = EMPTY;
    if (t == PAWN && u == ep) {
      b.sq[u + (white ? -8 : 8)] = EMPTY;
      cap = true;
    }
    if (t == KING && (u - s == 2 || s - u == 2)) {
      if (u > s) {
        b.sq[s + 1] = b.sq[s + 3];
        b.sq[s + 3] = EMPTY;
      } else {
        b.sq[s - 1] = b.sq[s - 4];
        b.sq[s - 4] = EMPTY;
      }
    }
    b.white = !white;
    uint8_t rights = castling;
    if (t == KING) rights &= white ? (uint8_t)~(CW_K | CW_Q) : (uint8_t)~(CB_K | CB_Q);
    const struct {
      int corner;
      uint8_t r;
    } corners[4] = {{0, CW_Q}, {7, CW_K}, {56, CB_Q}, {63, CB_K}};
    for (auto& c : corners)
      if (s == c.corner || u == c.corner) rights &= (uint8_t)~c.r;
    b.castling = rights;
    b.ep = (t == PAWN && (u - s == 16 || s - u == 16)) ? (int8_t)((s + u) / 2) : (int8_t)-1;
    b.halfmove = (t == PAWN || cap) ? 0 : halfmove + 1;
  }

  bool leaves_king_safe(const Move& mv) const {
    Board b;
    make(mv, b);
    const int k = b.king_square(white);
    return !b.attacked_by(k, !white);
  }

  static uint64_t between_mask(int a, int b) {
    const int fa = a & 7, ra = a >> 3, fb = b & 7, rb = b >> 3, df = fb - fa, dr = rb - ra;
    if (!(df == 0 || dr == 0 || df == dr || df == -dr)) return 0;
    const int sf = (df > 0) - (df < 0), sr = (dr > 0) - (dr < 0);
    uint64_t m = 0;
    int f = fa + sf, r = ra + sr;
    while (f != fb || r != rb) {
      m |= 1ull << (r * 8 + f);
      f += sf;
      r += sr;
    }
    return m;
  }

  void legal(std::vector<Move>& out) const {
    std::vector<Move> m;
    m.reserve(64);
    out.clear();
    if (!is_check()) {
      pseudo(m, ~0ull, true);
    } else {
      const int k = king_square(white);
      uint8_t tg[8];
      int n = 0;
      for (int i = 0; i < T.n_king[k]; ++i) tg[n++] = T.king[k][i];
      sort_desc(tg, n);
      for (int i = 0; i < n; ++i)
        if (!ours(sq[tg[i]])) m.push_back({(uint8_t)k, tg[i], 0});
      int ch[16];
      const int nc = checkers(ch);
      if (nc == 1) {
        const int c = ch[0];
        const uint64_t target = (1ull << c) | between_mask(k, c);
        pseudo(m, target, false);
        if (ep >= 0 && !((target >> ep) & 1)) {
          const int last_double = ep + (white ? -8 : 8);
          if (last_double == c) ep_moves(m);
        }
      }
    }
    for (const Move& mv : m)
      if (leaves_king_safe(mv)) out.push_back(mv);
  }

  uint64_t key() const {
    uint64_t h = white ? T.z_side : 0;
    for (int s = 0; s < 64; ++s)
      if (sq[s] != EMPTY) h ^= T.z_piece[sq[s]][s];
    h ^= T.z_castle[castling & 15];
    if (ep >= 0) {
      std::vector<Move> e;
      ep_moves(e);
      for (const Move& mv : e)
        if (leaves_king_safe(mv)) {
          h ^= T.z_ep[ep];
          break;
        }
    }
    return h;
  }

  bool insufficient(bool w) const {
    const uint8_t c = w ? 0 : BLACK;
    int n_ours = 0;
    bool knight = false, bishop = false;
    for (int s = 0; s < 64; ++s) {
      const uint8_t p = sq[s];
      if (p == EMPTY || (p & BLACK) != c) continue;
      ++n_ours;
      const int t = p & 7;
      if (t == PAWN || t == ROOK || t == QUEEN) return false;
      knight |= t == KNIGHT;
      bishop |= t == BISHOP;
    }
    if (knight) {
      if (n_ours > 2) return false;
      for (int s = 0; s < 64; ++s) {
        const uint8_t p = sq[s];
        if (p != EMPTY && (p & BLACK) != c && (p & 7) != KING && (p & 7) != QUEEN) return false;
      }
      return true;
    }
    if (bishop) {
      int colours = 0;
      for (int s = 0; s < 64; ++s) {
        const int t = sq[s] & 7;
        if (sq[s] == EMPTY) continue;
        if (t == PAWN || t == KNIGHT) return false;
        if (t == BISHOP) colours |= 1 << (((s & 7) + (s >> 3)) & 1);
      }
      return colours != 3;
    }
    return true;
  }

  // 0 ongoing; else termination * 4 + winner (0 draw, 1 white, 2 black);
  // terminations: 1 checkmate, 2 insufficient material, 3 stalemate,
  // 4 seventy-five moves, 5 fivefold repetition
  int outcome() const {
    std::vector<Move> m;
    legal(m);
    const bool has = !m.empty();
    if (!has && is_check()) return 1 * 4 + (white ? 2 : 1);
    if (insufficient(true) && insufficient(false)) return 2 * 4;
    if (!has) return 3 * 4;
    if (halfmove >= 150) return 4 * 4;
    if (!keys.empty()) {
      int n = 0;
      for (uint64_t k : keys) n += k == keys.back();
      if (n >= 5) return 5 * 4;
    }
    return 0;
  }
};

void start_position(Board& b) {
  const uint8_t back[8] = {ROOK, KNIGHT, BISHOP, QUEEN, KING, BISHOP, KNIGHT, ROOK};
  std::memset(b.sq, 0, 64);
  for (int f = 0; f < 8; ++f) {
    b.sq[f] = back[f];
    b.sq[8 + f] = PAWN;
    b.sq[48 + f] = PAWN | BLACK;
    b.sq[56 + f] = back[f] | BLACK;
  }
  b.white = true;
  b.castling = CW_K | CW_Q | CB_K | CB_Q;
  b.ep = -1;
  b.halfmove = 0;
  b.keys.assign(1, b.key());
}

int parse_sq(const char* t) {
  if (t[0] < 'a' || t[0] > 'h' || t[1] < '1' || t[1] > '8') return -1;
  return (t[0] - 'a') + 8 * (t[1] - '1');
}

int write_uci(const Move& m, char* o) {
  o[0] = (char)('a' + (m.from & 7));
  o[1] = (char)('1' + (m.from >> 3));
  o[2] = (char)('a' + (m.to & 7));
  o[3] = (char)('1' + (m.to >> 3));
  if (!m.promo) return 4;
  o[4] = "  nbrq"[m.promo];
  return 5;
}

uint64_t perft(const Board& b, int depth) {
  if (depth == 0) return 1;
  std::vector<Move> m;
  b.legal(m);
  if (depth == 1) return m.size();
  uint64_t n = 0;
  Board c;
  for (const Move& mv : m) {
    b.make(mv, c);
    n += perft(c, depth - 1);
  }
  return n;
}

}  // namespace

extern "C" {

void* allie_chess_start(void) {
  Board* b = new (std::nothrow) Board();
  if (b) start_position(*b);
  return b;
}

void* allie_chess_from_fen(const char* fen) {
  if (!fen) return nullptr;
  Board* b = new (std::nothrow) Board();
  if (!b) return nullptr;
  std::memset(b->sq, 0, 64);
  const char* p = fen;
  int r = 7, f = 0;
  for (; *p && *p != ' '; ++p) {
    const char ch = *p;
    if (ch == '/') {
      --r;
      f = 0;
      continue;
    }
    if (ch >= '1' && ch <= '8') {
      f += ch - '0';
      continue;
    }
    uint8_t t = 0;
    switch (ch | 0x20) {
      case 'p': t = PAWN; break;
      case 'n': t = KNIGHT; break;
      case 'b': t = BISHOP; break;
      case 'r': t = ROOK; break;
      case 'q': t = QUEEN; break;
      case 'k': t = KING; break;
      default: delete b; return nullptr;
    }
    if (r < 0 || f > 7) {
      delete b;
      return nullptr;
    }
    b->sq[r * 8 + f] = (uint8_t)(t | ((ch >= 'a') ? BLACK : 0));
    ++f;
  }
  while (*p == ' ') ++p;
  b->white = *p != 'b';
  while (*p && *p != ' ') ++p;
  while (*p == ' ') ++p;
  b->castling = 0;
  for (; *p && *p != ' '; ++p) {
    if (*p == 'K') b->castling |= CW_K;
    if (*p == 'Q') b->castling |= CW_Q;
    if (*p == 'k') b->castling |= CB_K;
    if (*p == 'q') b->castling |= CB_Q;
  }
  while (*p == ' ') ++p;
  b->ep = -1;
  if (*p && *p != '-' && p[1]) b->ep = (int8_t)parse_sq(p);
  while (*p && *p != ' ') ++p;
  while (*p == ' ') ++p;
  b->halfmove = *p ? std::atoi(p) : 0;
  if (b->king_square(true) < 0 || b->king_square(false) < 0) {
    delete b;
    return nullptr;
  }
  b->keys.assign(1, b->key());
  return b;
}

void allie_chess_free(void* b) { delete static_cast<Board*>(b); }

// the position after a legal UCI move, or null (illegal or malformed move)
void* allie_chess_push_uci(const void* bp, const char* uci) {
  const Board& b = *static_cast<const Board*>(bp);
  const size_t n = uci ? std::strlen(uci) : 0;
  if (n != 4 && n != 5) return nullptr;
  const int s = parse_sq(uci), u = parse_sq(uci + 2);
  if (s < 0 || u < 0) return nullptr;
  uint8_t promo = 0;
  if (n == 5) {
    switch (uci[4]) {
      case 'q': promo = QUEEN; break;
      case 'r': promo = ROOK; break;
      case 'b': promo = BISHOP; break;
      case 'n': promo = KNIGHT; break;
      default: return nullptr;
    }
  }
  std::vector<Move> m;
  b.legal(m);
  for (const Move& mv : m) {
    if (mv.from != s || mv.to != u || mv.promo != promo) continue;
    Board* c = new (std::nothrow) Board();
    if (!c) return nullptr;
    b.make(mv, *c);
    if (c->halfmove == 0) {
      c->keys.assign(1, c->key());
    } else {
      c->keys.reserve(b.keys.size() + 1);
      c->keys = b.keys;
      c->keys.push_back(c->key());
    }
    return c;
  }
  return nullptr;
}

// legal moves as space-separated UCI (NUL-terminated) in the generation
// order; returns the count, or -(bytes needed) when cap is too small
int allie_chess_legal_uci(const void* bp, char* out, int cap) {
  const Board& b = *static_cast<const Board*>(bp);
  std::vector<Move> m;
  b.legal(m);
  char buf[8];
  int need = 1;
  for (const Move& mv : m) need += write_uci(mv, buf) + 1;
  if (need > cap) return -need;
  int o = 0;
  for (size_t i = 0; i < m.size(); ++i) {
    if (i) out[o++] = ' ';
    o += write_uci(m[i], out + o);
  }
  out[o] = 0;
  return (int)m.size();
}

int allie_chess_outcome(const void* bp) { return static_cast<const Board*>(bp)->outcome(); }

int allie_chess_is_check(const void* bp) { return static_cast<const Board*>(bp)->is_check() ? 1 : 0; }

int allie_chess_white_to_move(const void* bp) { return static_cast<const Board*>(bp)->white ? 1 : 0; }

long long allie_chess_perft(const void* bp, int depth) {
  return (long long)perft(*static_cast<const Board*>(bp), depth);
}

}  // extern "C"
