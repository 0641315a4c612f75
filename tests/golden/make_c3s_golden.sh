#!/bin/sh
# make_c3s_golden.sh - writes the long-context fixtures of the model with
# Qwen3-30B-A3B's attention geometry (oracle/make_c3s.sh builds it with the
# reference's own tools):
#   c3s_greedy.txt   the reference's 128 greedy tokens after a 1920-token
#                    xorshift(42) prompt (tierlm run --print-tokens)
#   c3s_oracle.jsonl its top-10 logits at every one of the 2047 positions of
#                    prompt + the first 127 greedy tokens, teacher-forced
#                    (tierlm oracle)
# Run here, where the reference's tools are built; the fixtures are data.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
B="$ROOT/oracle/_ref/bin"
S="$ROOT/oracle/_ref/c3s"
[ -f "$S/c3s.tlmm" ] || sh "$ROOT/oracle/make_c3s.sh"
PROMPT=$(python3 -c "
x, out, M = 42, [], (1 << 64) - 1
for i in range(1920):
    x ^= (x << 13) & M; x ^= x >> 7; x ^= (x << 17) & M
    out.append(x % 2048)
print(','.join(map(str, out)))")
"$B/tierlm" run "$S/c3s.tlmm" --tokens "$PROMPT" -n 128 --print-tokens --cache 1G 2>/dev/null > "$HERE/c3s_greedy.txt"
GEN=$(tr ' ' ',' < "$HERE/c3s_greedy.txt" | cut -d, -f1-127)
"$B/tierlm" oracle "$S/c3s.tlmm" --tokens "$PROMPT,$GEN" --cache 1G 2>/dev/null > "$HERE/c3s_oracle.jsonl"
