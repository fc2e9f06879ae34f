// resident.js -- the resident harness's correctness commands over the JS host
// (resident-a4b.html:96-101 and its runCmd branches, :115-206):
//   node resident.js <model.gguf> <goldens.json> gate [n] [p]   generateFast vs the goldens' greedy ids
//   node resident.js <model.gguf> <goldens.json> gate2 [n] [p]  the same after the batched prefill
//   node resident.js <model.gguf> <goldens.json> stats          per-layer hidden meanAbs of prompt 0
// A goldens file is JSON {"prompts": [{"input_ids": [...], "generated_ids":
// [...]}, ...]} (the layout of goldens/goldens-a4b.json).  Lines as the
// reference logs them: "[p<i>] MATCH|MISMATCH got=[...] want=[...]", the first
// divergence, "GATE PASS|FAIL"; "embed: meanAbs=... first4=[...]",
// "layer<l>: meanAbs=... first4=[...]" (stopping at a non-finite layer).  The
// exit code is 0 on a pass (all layers finite for stats).
"use strict";
const fs = require("fs");
const { loadEngine, FLAG_LAYER_HIDDEN } = require("./engine");
const { openGGUF } = require("./gguf");

// IEEE half -> number
function f16(h) {
  const s = h & 0x8000 ? -1 : 1, e = (h >> 10) & 31, m = h & 1023;
  if (e === 0) return s * m * Math.pow(2, -24);
  if (e === 31) return m ? NaN : s * Infinity;
  return s * (1024 + m) * Math.pow(2, e - 25);
}

// row `row` of a raw ggml Q6_K matrix [rows][cols] (per 256 weights: ql[128]
// low nibbles, qh[64] high bit pairs, 16 int8 scales, f16 d; weight =
// d * scale * (q - 32) in ggml's element order)
function q6kRow(buf, cols, row) {
  const nsb = cols / 256, out = new Float32Array(cols);
  for (let b = 0; b < nsb; b++) {
    const o = (row * nsb + b) * 210;
    const d = f16(buf[o + 208] | (buf[o + 209] << 8));
    for (let half = 0; half < 2; half++) {
      const ql = o + 64 * half, qh = o + 128 + 32 * half, sc = o + 192 + 8 * half;
      for (let l = 0; l < 32; l++) {
        const h = buf[qh + l], lo = buf[ql + l], hi = buf[ql + l + 32];
        const q = [(lo & 15) | ((h & 3) << 4), (hi & 15) | (((h >> 2) & 3) << 4),
                   (lo >> 4) | (((h >> 4) & 3) << 4), (hi >> 4) | (((h >> 6) & 3) << 4)];
        for (let j = 0; j < 4; j++) {
          const s = (buf[sc + 2 * j + (l >> 4)] << 24) >> 24;  // int8
          out[256 * b + 128 * half + 32 * j + l] = d * s * (q[j] - 32);
        }
      }
    }
  }
  return out;
}

async function gate(eng, goldens, n = 24, p = undefined, batched = false, log = console.log) {
  let allPass = true;
  for (let pi = 0; pi < goldens.prompts.length; pi++) {
    if (p !== undefined && pi !== p) continue;
    const g = goldens.prompts[pi];
    const want = g.generated_ids.slice(0, n);
    const got = batched ? await eng.generatePrefill(g.input_ids, want.length)
                        : await eng.generateFast(g.input_ids, want.length);
    const match = got.length === want.length && got.every((t, i) => t === want[i]);
    allPass = allPass && match;
    log(`[p${pi}] ${match ? "MATCH" : "MISMATCH"} got=${JSON.stringify(got)} want=${JSON.stringify(want)}`);
    if (!match) {
      let first = -1;
      for (let i = 0; i < Math.max(got.length, want.length); i++)
        if (i >= got.length || i >= want.length || got[i] !== want[i]) { first = i; break; }
      log(`[p${pi}] first divergence at ${first}`);
    }
  }
  log((batched ? "GATE2 " : "GATE ") + (allPass ? "PASS" : "FAIL"));
  return allPass;
}

function line(name, h) {
  let s = 0;
  for (const v of h) s += Math.abs(v);
  return { name, meanAbs: s / h.length, first4: Array.from(h.slice(0, 4)) };
}

// per-layer hidden meanAbs of prompt 0's last token; embd = the raw Q6_K
// bytes of token_embd.weight (or null), hidden = the model width
async function stats(eng, goldens, embd, hidden, layers, log = console.log) {
  const ids = goldens.prompts[0].input_ids;
  for (let pos = 0; pos < ids.length - 1; pos++) await eng.step(ids[pos], pos);
  await eng.step(ids[ids.length - 1], ids.length - 1);
  const out = [];
  if (embd) {
    const e = q6kRow(embd, hidden, ids[ids.length - 1]);
    const m = Math.fround(Math.sqrt(hidden));
    out.push(line("embed", e.map((v) => Math.fround(v * m))));
  }
  for (let l = 0; l < layers; l++) out.push(line(`layer${l}`, await eng.readLayerHidden(l)));
  for (const r of out) {
    log(`${r.name}: meanAbs=${r.meanAbs.toFixed(4)} first4=${JSON.stringify(r.first4.map((x) => Number(x.toFixed(4))))}`);
    if (!isFinite(r.meanAbs)) break;
  }
  return out;
}

async function main() {
  const [file, goldensPath, mode, a1, a2] = process.argv.slice(2);
  if (!file || !goldensPath || !["gate", "gate2", "stats"].includes(mode)) {
    console.error("usage: node resident.js model.gguf goldens.json gate|gate2|stats [n] [p]");
    process.exit(2);
  }
  const goldens = JSON.parse(fs.readFileSync(goldensPath, "utf8"));
  if (!goldens || !Array.isArray(goldens.prompts)) throw new Error(`${goldensPath}: no 'prompts' list`);
  const eng = await loadEngine(file, { flags: FLAG_LAYER_HIDDEN });
  let ok;
  if (mode === "stats") {
    const g = openGGUF(file);
    const emb = await g.fetch("token_embd.weight");
    g.close();
    const res = await stats(eng, goldens, emb.buf, emb.dims[0], eng.C.layers);
    ok = res.every((r) => isFinite(r.meanAbs));
  } else {
    ok = await gate(eng, goldens, a1 !== undefined ? Number(a1) : 24, a2 !== undefined ? Number(a2) : undefined,
                    mode === "gate2");
  }
  eng.close();
  process.exit(ok ? 0 : 1);
}

module.exports = { gate, stats, q6kRow, f16 };
if (require.main === module) {
  main().catch((e) => {
    console.error(e && e.stack ? e.stack : String(e));
    process.exit(1);
  });
}
