#!/bin/sh
# make_c5s.sh - TEST INFRASTRUCTURE ONLY: a synthetic model with the
# attention grouping of Qwen3-235B-A22B (16 query heads per key head of
# width 128) at a small size: 2 layers, D 2048, 32 query / 2 key heads of
# width 128, qk-norm, rope theta 1e6, context capacity 4096 (the
# synthesiser's max_position_embeddings), 16 experts top-8 of width 256 in
# Q4_K (the 235B configuration's expert format) under the softmax router, no
# shared expert, Q8_0 dense, vocabulary 2048, seed 13.  Written by the
# reference's own tools (built from its sources by `make -C oracle tools`)
# into oracle/_ref/c5s:
#   c5s.tlmm, d0/   tlmc compile --profile exact --experts q4_k
# with the SHA-256 of the synth output checked against the values recorded
# when this fixture was first made.  Nothing here is copied from the reference.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
B="$HERE/_ref/bin"
O="$HERE/_ref/c5s"
[ -x "$B/tlmc" ] && [ -x "$B/tierlm" ] || make -C "$HERE" tools >/dev/null
rm -rf "$O"
mkdir -p "$O/d0"
"$B/tlmc" synth --out "$O/src" --layers 2 --d-model 2048 --heads 32 --kv-heads 2 --head-dim 128 \
    --experts 16 --top-k 8 --d-expert 256 --shared 0 --vocab 2048 --seed 13 > "$O/synth.log" 2>&1
echo "3d093a9c3a2d6f4d6969aff88d7d97eea55c5985d8a9a732fba75e91b481db6b  $O/src/model.safetensors" | sha256sum -c -
echo "5e72a45a202f725cde91e93f6d54bf71aaf00a0ee686038cd54215a45bca9816  $O/src/config.json" | sha256sum -c -
"$B/tlmc" compile "$O/src" --out "$O/c5s.tlmm" --drives "$O/d0" --profile exact --experts q4_k \
    > "$O/compile.log" 2>&1
rm -rf "$O/src" "$O/c5s.work"
