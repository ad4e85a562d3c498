#!/bin/bash
# Regenerates mt19937_kat.json from the C++ standard library (g++ / libstdc++).
set -e
cd "$(dirname "$0")"
tmp=$(mktemp -d)
g++ -O2 -std=c++17 -o "$tmp/kat" mt19937_kat.cpp
"$tmp/kat" > mt19937_kat.json
rm -rf "$tmp"
python3 -c "import json; d = json.load(open('mt19937_kat.json')); print('ok', d['default_10000th'])"
