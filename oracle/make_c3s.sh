#!/bin/sh
# make_c3s.sh - TEST INFRASTRUCTURE ONLY: a synthetic model with the attention
# geometry of Qwen3-30B-A3B and a small expert count, for the device decode
# step at long contexts: 2 layers, D 2048, 32 query / 4 key heads of width
# 128, qk-norm, rope theta 1e6, context capacity 4096 (the synthesiser's
# max_position_embeddings), 16 experts top-8 of width 256 (Q6_K) under the
# softmax router, no shared expert, Q8_0 dense, vocabulary 2048, seed 11.
# Written by the reference's own tools (built from its sources by
# `make -C oracle tools`) into oracle/_ref/c3s:
#   c3s.tlmm, d0/   tlmc compile --profile exact
# with the SHA-256 of the synth output checked against the values recorded
# when this fixture was first made.  Nothing here is copied from the reference.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
B="$HERE/_ref/bin"
O="$HERE/_ref/c3s"
[ -x "$B/tlmc" ] && [ -x "$B/tierlm" ] || make -C "$HERE" tools >/dev/null
rm -rf "$O"
mkdir -p "$O/d0"
"$B/tlmc" synth --out "$O/src" --layers 2 --d-model 2048 --heads 32 --kv-heads 4 --head-dim 128 \
    --experts 16 --top-k 8 --d-expert 256 --shared 0 --vocab 2048 --seed 11 > "$O/synth.log" 2>&1
echo "a82005b064a94d84749cab5aec414a63d32110f459f8c56f5bf03390ef361a8c  $O/src/model.safetensors" | sha256sum -c -
echo "301c1fc6bfb4f7a52000cec72ad9e784e5c771ca5ddc09fe14f46af4346e2112  $O/src/config.json" | sha256sum -c -
"$B/tlmc" compile "$O/src" --out "$O/c3s.tlmm" --drives "$O/d0" --profile exact > "$O/compile.log" 2>&1
rm -rf "$O/src" "$O/c3s.work"
