#!/bin/sh
# make_c3s_long_golden.sh - TEST INFRASTRUCTURE ONLY: the reference's own
# runtime on the C3S store (oracle/make_c3s.sh, context capacity 4096) past
# 2048 positions: a 2300-token xorshift(42) prompt (vocabulary 2048) and the
# 48 greedy tokens after it (`tierlm run --print-tokens`), into
# tests/golden/c3s_long_greedy.txt.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
S="$ROOT/oracle/_ref/c3s"
[ -f "$S/c3s.tlmm" ] || sh "$ROOT/oracle/make_c3s.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(2300):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 2048)
print(','.join(map(str, out)))")
"$B/tierlm" run "$S/c3s.tlmm" --tokens "$PROMPT" -n 48 --print-tokens --cache 1G 2>/dev/null > "$HERE/c3s_long_greedy.txt"
