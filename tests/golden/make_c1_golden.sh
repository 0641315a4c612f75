#!/bin/sh
# make_c1_golden.sh - writes the end-to-end fixtures of the 4-layer synthetic
# model (oracle/make_c1.sh builds it with the reference's own tools):
#   c1_greedy.txt   the reference's 64 greedy tokens after the 64-token
#                   xorshift(42) prompt (tierlm run --print-tokens)
#   c1_oracle.jsonl its top-10 logits at every position of prompt + the first
#                   63 greedy tokens, teacher-forced (tierlm oracle)
#   c1_greedy_long.txt  320 greedy tokens after the same prompt (positions up
#                   to 383: several attention chunks and score passes)
#   c1_oracle_long.jsonl  top-10 logits at every position of prompt + the
#                   first 319 of those tokens, teacher-forced
# Run here, where the reference's tools are built; the fixtures are data.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
C1="$ROOT/oracle/_ref/c1"
[ -f "$C1/c1.tlmm" ] || sh "$ROOT/oracle/make_c1.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(64):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 4096)
print(','.join(map(str, out)))")
"$B/tierlm" run "$C1/c1.tlmm" --tokens "$PROMPT" -n 64 --print-tokens --cache 1G 2>/dev/null > "$HERE/c1_greedy.txt"
echo "f2fb519981d61a8626b130207ac434f1  $HERE/c1_greedy.txt" | md5sum -c -
GEN=$(tr ' ' ',' < "$HERE/c1_greedy.txt" | cut -d, -f1-63)
"$B/tierlm" oracle "$C1/c1.tlmm" --tokens "$PROMPT,$GEN" --cache 1G 2>/dev/null > "$HERE/c1_oracle.jsonl"
"$B/tierlm" run "$C1/c1.tlmm" --tokens "$PROMPT" -n 320 --print-tokens --cache 1G 2>/dev/null > "$HERE/c1_greedy_long.txt"
GENL=$(tr ' ' ',' < "$HERE/c1_greedy_long.txt" | cut -d, -f1-319)
"$B/tierlm" oracle "$C1/c1.tlmm" --tokens "$PROMPT,$GENL" --cache 1G 2>/dev/null > "$HERE/c1_oracle_long.jsonl"
