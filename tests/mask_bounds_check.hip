// Host-side check of the interval masks of probjax_amd/csrc/attn_mods.h:
// row_bounds and key_bounds against the masks' element-wise definitions
// (probjax/nn/pallas_kernels/attention_mask_bias.py), on random
// combinations of causal shift, windows, prefix and sequence lengths, KV
// lengths and static lengths.  Built for the host only and run by
// tests/test_mask_bounds.py; prints "ok <cases>" or the first mismatch.
#include <cstdio>
#include <cstdlib>

#include "../probjax_amd/csrc/attn_mods.h"

using namespace pjx;

static int rnd(int n) { return std::rand() % n; }

int main() {
  std::srand(12345);
  long checked = 0;
  for (int it = 0; it < 4000; ++it) {
    const int Lq = 1 + rnd(40), Lk = 1 + rnd(40);
    int32_t prefix = rnd(Lk + 3) - 1, seqlen = rnd(Lq + 5) - 1, kvlen = rnd(Lk + 3) - 1;
    ScoreMods m{};
    const bool causal = rnd(2);
    m.causal_shift = causal ? rnd(2 * Lk + 1) - Lk : 0;
    m.win_left = rnd(3) ? kNoBound : rnd(Lk + 2);
    m.win_right = rnd(3) ? kNoBound : rnd(Lk + 2);
    m.prefix = rnd(3) ? nullptr : &prefix;
    m.seqlen = rnd(3) ? nullptr : &seqlen;
    const bool use_kvlen = rnd(2);
    const int q_valid = rnd(3) ? Lq : rnd(Lq + 1), kv_valid = rnd(3) ? Lk : rnd(Lk + 1);
    int kv_end = kv_valid < Lk ? kv_valid : Lk;
    if (use_kvlen) kv_end = kv_end < (kvlen > 0 ? kvlen : 0) ? kv_end : (kvlen > 0 ? kvlen : 0);
    const int q_hi = q_valid;
    for (int q = 0; q < Lq; ++q) {
      int lo, hi;
      row_bounds(m, causal, 0, kv_end, q_hi, q, lo, hi);
      for (int k = 0; k < Lk; ++k) {
        bool want = q < q_hi && k < kv_end;
        if (causal) want = want && k <= q + m.causal_shift;
        if (m.win_left != kNoBound) want = want && q - k <= m.win_left;
        if (m.win_right != kNoBound) want = want && k - q <= m.win_right;
        if (m.prefix) want = want && (k < prefix || q >= k);
        if (m.seqlen) want = want && ((q < seqlen && k < seqlen) || q == k);
        const bool row = lo <= k && k <= hi;
        int qlo, qhi;
        key_bounds(m, causal, 0, kv_end, q_hi, k, qlo, qhi);
        const bool col = qlo <= q && q <= qhi;
        if (row != want || col != want) {
          std::printf("mismatch it=%d q=%d k=%d want=%d row=%d col=%d causal=%d shift=%d wl=%d wr=%d "
                      "prefix=%d seqlen=%d kv_end=%d q_hi=%d\n",
                      it, q, k, want, row, col, causal, m.causal_shift, m.win_left, m.win_right,
                      m.prefix ? prefix : -99, m.seqlen ? seqlen : -99, kv_end, q_hi);
          return 1;
        }
        ++checked;
      }
    }
    // monotone ends: the tile ranges rely on them
    int plo = -(1 << 30), phi = -(1 << 30);
    for (int q = 0; q < q_hi && q < Lq; ++q) {
      int lo, hi;
      row_bounds(m, causal, 0, kv_end, q_hi, q, lo, hi);
      if (lo < plo || hi < phi) {
        std::printf("non-monotone row bounds it=%d q=%d\n", it, q);
        return 1;
      }
      plo = lo;
      phi = hi;
    }
  }
  std::printf("ok %ld\n", checked);
  return 0;
}
