#!/bin/sh
# make_c6d_golden.sh - writes the fixtures of the model with two leading
# dense-FFN layers (oracle/make_c6d.sh builds it with the reference's own
# tools):
#   c6d_greedy.txt   the reference's 64 greedy tokens after a 200-token
#                    xorshift(42) prompt (tierlm run --print-tokens)
#   c6d_oracle.jsonl its top-10 logits at every one of the 263 positions of
#                    prompt + the first 63 greedy tokens, teacher-forced
#                    (tierlm oracle)
# Run here, where the reference's tools are built; the fixtures are data.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
S="$ROOT/oracle/_ref/c6d"
[ -f "$S/c6d.tlmm" ] || sh "$ROOT/oracle/make_c6d.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(200):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 2048)
print(','.join(map(str, out)))")
"$B/tierlm" run "$S/c6d.tlmm" --tokens "$PROMPT" -n 64 --print-tokens --cache 1G 2>/dev/null > "$HERE/c6d_greedy.txt"
GEN=$(tr ' ' ',' < "$HERE/c6d_greedy.txt" | cut -d, -f1-63)
"$B/tierlm" oracle "$S/c6d.tlmm" --tokens "$PROMPT,$GEN" --cache 1G 2>/dev/null > "$HERE/c6d_oracle.jsonl"
