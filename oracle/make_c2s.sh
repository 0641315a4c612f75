#!/bin/sh
# make_c2s.sh - TEST INFRASTRUCTURE ONLY: a second synthetic model for the
# device decode step, shaped to reach what the 4-layer model (make_c1.sh) does
# not: 2 layers, D 256, 4 query / 2 key heads of width 128, no qk-norm, YaRN
# RoPE (x4 over 1024), 16 experts top-2 under the sigmoid router (selection
# bias, routed scale 2.5), no shared expert, Q4_K experts, vocabulary 2048,
# seed 7.  Written by the reference's own tools (built from its sources by
# `make -C oracle tools`) into oracle/_ref/c2s:
#   c2s.tlmm, d0/   tlmc compile --profile exact --experts q4_k
# with the SHA-256 of the synth output checked against the values recorded
# when this fixture was first made.  Nothing here is copied from the reference.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
B="$HERE/_ref/bin"
O="$HERE/_ref/c2s"
[ -x "$B/tlmc" ] && [ -x "$B/tierlm" ] || make -C "$HERE" tools >/dev/null
rm -rf "$O"
mkdir -p "$O/d0"
"$B/tlmc" synth --out "$O/src" --layers 2 --d-model 256 --heads 4 --kv-heads 2 --head-dim 128 \
    --experts 16 --top-k 2 --d-expert 256 --shared 0 --vocab 2048 --seed 7 --router sigmoid --qk-norm no \
    --yarn > "$O/synth.log" 2>&1
echo "93a1b452d91c8263b1a6c7524c0ed9465995d5f9a481810fb578b9c36ba4a90e  $O/src/model.safetensors" | sha256sum -c -
echo "ee010944d8d89ae47a5a0810dbcb96a115f9c072bdf702101ab065a9ab920257  $O/src/config.json" | sha256sum -c -
"$B/tlmc" compile "$O/src" --out "$O/c2s.tlmm" --drives "$O/d0" --profile exact --experts q4_k \
    > "$O/compile.log" 2>&1
rm -rf "$O/src" "$O/c2s.work"
