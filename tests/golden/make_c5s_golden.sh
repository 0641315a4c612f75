#!/bin/sh
# make_c5s_golden.sh - writes the fixtures of the model with Qwen3-235B-A22B's
# attention grouping, 16 query heads per key head (oracle/make_c5s.sh builds
# it with the reference's own tools):
#   c5s_greedy.txt   the reference's 64 greedy tokens after a 1100-token
#                    xorshift(42) prompt (tierlm run --print-tokens)
#   c5s_oracle.jsonl its top-10 logits at every one of the 1163 positions of
#                    prompt + the first 63 greedy tokens, teacher-forced
#                    (tierlm oracle)
# Run here, where the reference's tools are built; the fixtures are data.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
S="$ROOT/oracle/_ref/c5s"
[ -f "$S/c5s.tlmm" ] || sh "$ROOT/oracle/make_c5s.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(1100):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 2048)
print(','.join(map(str, out)))")
"$B/tierlm" run "$S/c5s.tlmm" --tokens "$PROMPT" -n 64 --print-tokens --cache 1G 2>/dev/null > "$HERE/c5s_greedy.txt"
GEN=$(tr ' ' ',' < "$HERE/c5s_greedy.txt" | cut -d, -f1-63)
"$B/tierlm" oracle "$S/c5s.tlmm" --tokens "$PROMPT,$GEN" --cache 1G 2>/dev/null > "$HERE/c5s_oracle.jsonl"
