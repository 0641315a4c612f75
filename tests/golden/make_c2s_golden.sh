#!/bin/sh
# make_c2s_golden.sh - writes the end-to-end fixtures of the second synthetic
# model (oracle/make_c2s.sh builds it with the reference's own tools):
#   c2s_greedy.txt   the reference's 64 greedy tokens after the 64-token
#                    xorshift(42) prompt (tierlm run --print-tokens)
#   c2s_oracle.jsonl its top-10 logits at every position of prompt + the
#                    first 63 greedy tokens, teacher-forced (tierlm oracle)
# Run here, where the reference's tools are built; the fixtures are data.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
S="$ROOT/oracle/_ref/c2s"
[ -f "$S/c2s.tlmm" ] || sh "$ROOT/oracle/make_c2s.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(64):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 2048)
print(','.join(map(str, out)))")
"$B/tierlm" run "$S/c2s.tlmm" --tokens "$PROMPT" -n 64 --print-tokens --cache 1G 2>/dev/null > "$HERE/c2s_greedy.txt"
GEN=$(tr ' ' ',' < "$HERE/c2s_greedy.txt" | cut -d, -f1-63)
"$B/tierlm" oracle "$S/c2s.tlmm" --tokens "$PROMPT,$GEN" --cache 1G 2>/dev/null > "$HERE/c2s_oracle.jsonl"
