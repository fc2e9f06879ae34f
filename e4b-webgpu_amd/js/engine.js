// engine.js -- the JS host of the MI355X decode engine.  loadEngine(path)
// opens a GGUF file (gguf.js), uploads every tensor through the N-API addon
// into libe4b.so (which repacks and owns the device copies) and returns an
// object with the surface of the one loadEngineA4B returns
// (src/engine-a4b.js:854-856): step(token, pos), argmaxFast(),
// decodeChunk(startPos, count, ringBase), generateFast(ids, maxNew, eosIds),
// prefill(ids), generatePrefill(ids, maxNew, eosIds), profileStep(token,
// pos), profilePrefill(ids), readHidden(), readLayerHidden(layer); the long-context pair compactAll() and
// generateLong(ids, maxNew, eosIds) (src/engine-a4b.js:587-657, with
// FLAG_KV_SCORE); plus readLogits(), kvCount(), reset() and close().
//
// The GPU work runs in libe4b.so; the async functions resolve when the call
// has returned (every library call that returns results is synchronous).
"use strict";
const path = require("path");
const { openGGUF } = require("./gguf");

const addon = require(path.join(__dirname, "e4b_napi.node"));

// GGUF metadata keys of the E4B-shaped model (architecture prefix "e4b")
const KV = {
  hidden: "embedding_length", layers: "block_count", qHeads: "attention.head_count",
  kvHeads: "attention.head_count_kv", headDim: "attention.key_length", ffn: "feed_forward_length",
  pleDim: "embedding_length_per_layer_input", vocab: "vocab_size", window: "attention.sliding_window",
  ropeAngles: "rope.dimension_count_half", thetaLocal: "rope.freq_base_swa", thetaGlobal: "rope.freq_base",
  eps: "attention.layer_norm_rms_epsilon", softcap: "final_logit_softcapping",
};
const DEFAULTS = { ring: 1024, maxSeq: 4096, attnChunk: 0, maxPrompt: 0, flags: 0 };
const FLAG_NO_GRAPH = 1, FLAG_STEP_PREFILL = 2, FLAG_KV_SCORE = 4, FLAG_LAYER_HIDDEN = 16;
// long-context constants (src/engine-a4b.js:18-20)
const KV_BUDGET = 640, KV_DECAP = 768, KV_PROTECT = 64;

// the gemma4 MoE keys loadEngineA4B reads (src/engine-a4b.js:100-116): the
// A4B recipe (recipe 1) -- head dims key_length (full) / key_length_swa
// (sliding), KV heads per layer, a quarter of the full layers' pairs
// rotated, theta 1e4 / 1e6 (:329), the ring window + 512 slots (:198)
const KV_A4B = {
  hidden: "embedding_length", layers: "block_count", qHeads: "attention.head_count",
  ffn: "feed_forward_length", expertFfn: "expert_feed_forward_length", nExperts: "expert_count",
  window: "attention.sliding_window", eps: "attention.layer_norm_rms_epsilon", softcap: "final_logit_softcapping",
  headDimFull: "attention.key_length", headDim: "attention.key_length_swa", vocab: "vocab_size",
};
const RECIPE_A4B = 1, TOP_K = 8;

function configFromKVA4B(kv, arch, overrides) {
  const C = Object.assign({}, DEFAULTS, { recipe: RECIPE_A4B, pleDim: 0 });
  for (const [f, k] of Object.entries(KV_A4B)) {
    const key = `${arch}.${k}`;
    if (kv[key] !== undefined) C[f] = kv[key];
  }
  const used = kv[`${arch}.expert_used_count`];
  if (used !== undefined && used !== TOP_K) throw new Error(`expert_used_count ${used} (the MoE kernels select ${TOP_K})`);
  const kvh = kv[`${arch}.attention.head_count_kv`];
  if (Array.isArray(kvh)) {
    C.layerKvHeads = kvh.map(Number);
    C.kvHeads = C.layerKvHeads[0];
  }
  const pat = kv[`${arch}.attention.sliding_window_pattern`];
  if (pat !== undefined) C.layerGlobal = pat.map((s) => (s ? 0 : 1));
  Object.assign(C, overrides);
  C.ropeAngles = C.headDim / 2;
  C.ropeAnglesFull = Math.floor((0.25 * C.headDimFull) / 2);
  C.thetaLocal = 10000.0;
  C.thetaGlobal = 1000000.0;
  C.ring = Math.max(C.ring, C.window + 512);
  if (!C.layerGlobal) C.layerGlobal = Array.from({ length: C.layers }, (_, i) => (i % 6 === 5 ? 1 : 0));
  return C;
}

function configFromKV(kv, overrides = {}) {
  const arch = kv["general.architecture"] || "e4b";
  if (kv[`${arch}.expert_count`] !== undefined) return configFromKVA4B(kv, arch, overrides);
  const C = Object.assign({}, DEFAULTS);
  for (const [f, k] of Object.entries(KV)) {
    const key = `${arch}.${k}`;
    if (kv[key] !== undefined) C[f] = kv[key];
  }
  const pat = kv[`${arch}.attention.sliding_window_pattern`];
  if (pat !== undefined) C.layerGlobal = pat.map((s) => (s ? 0 : 1));
  Object.assign(C, overrides);
  if (!C.layerGlobal) C.layerGlobal = Array.from({ length: C.layers }, (_, i) => (i % 5 === 4 ? 1 : 0));
  return C;
}

async function loadEngine(file, overrides = {}) {
  const g = openGGUF(file);
  const arch = g.kv["general.architecture"] || "e4b";
  const emb = g.tensors["token_embd.weight"];
  if (g.kv[`${arch}.vocab_size`] === undefined && emb && emb.dims.length >= 2 && overrides.vocab === undefined)
    overrides = Object.assign({}, overrides, { vocab: Number(emb.dims[1]) });  // the embedding's row count
  const C = configFromKV(g.kv, overrides);
  const ctx = addon.create(C);
  try {
    for (const name of Object.keys(g.tensors)) {
      const t = await g.fetch(name);
      addon.setTensor(ctx, name, t.type, t.dims, t.buf);
    }
    addon.finalize(ctx);
  } catch (e) {
    addon.destroy(ctx);
    throw e;
  } finally {
    g.close();
  }
  const tokRing = [];

  async function step(token, pos) {
    return addon.step(ctx, token, pos, false).argmax;
  }
  async function argmaxFast() {
    return addon.argmax(ctx);
  }
  // GPU-fed greedy decode of `count` tokens from startPos, each fed with the
  // previous argmax; the tokens land in the host token ring at ringBase
  function decodeChunk(startPos, count, ringBase = 0) {
    const toks = addon.decode(ctx, startPos, count);
    for (let i = 0; i < count; i++) tokRing[ringBase + i] = toks[i];
    return toks;
  }
  async function prefill(inputIds) {
    return addon.prefill(ctx, Uint32Array.from(inputIds));
  }
  // src/engine-a4b.js:826-848: the prompt through the decode step token by
  // token, then GPU-fed chunks of <= 8 tokens with an EOS check after each
  // chunk's readback
  async function generateFast(inputIds, maxNew, eosIds = new Set([106, 1])) {
    return decodeLoop(addon.prefillSteps(ctx, Uint32Array.from(inputIds)), inputIds.length, maxNew, eosIds);
  }
  // src/engine-a4b.js:659-681: the batched prefill, then the same loop
  async function generatePrefill(inputIds, maxNew, eosIds = new Set([106, 1])) {
    return decodeLoop(await prefill(inputIds), inputIds.length, maxNew, eosIds);
  }
  // per-dispatch GPU budget, summed per kernel role (ranking only):
  // profileStep (src/engine-a4b.js:707-741) runs a real step,
  // profilePrefill (:743-779) one batched-prefill chunk of the first <= 512
  // tokens; both return a Map role -> {us, n} as the reference does
  const toMap = (arr) => new Map(arr.map((e) => [e.name, { us: e.us, n: e.n }]));
  async function profileStep(token, pos) {
    return toMap(addon.profileStep(ctx, token, pos));
  }
  async function profilePrefill(inputIds) {
    return toMap(addon.profilePrefill(ctx, Uint32Array.from(inputIds)));
  }
  function decodeLoop(g0, nPrompt, maxNew, eosIds) {
    const out = [g0];
    if (eosIds.has(g0)) return out;
    let pos = nPrompt, done = 1;
    while (done < maxNew) {
      const n = Math.min(8, maxNew - done);
      const toks = decodeChunk(pos, n, done - 1);
      pos += n;
      let stop = false;
      for (let k = 0; k < n; k++) {
        out.push(toks[k]);
        if (eosIds.has(toks[k])) { stop = true; break; }
      }
      done += n;
      if (stop) break;
    }
    return out.slice(0, maxNew);
  }
  // budget compaction of the full layers (src/engine-a4b.js:587-617): the
  // library ranks the accumulated attention mass, keeps the top entries plus
  // the newest `protect`, gathers them and zeroes the scores
  async function compactAll(budget = KV_BUDGET, protect = KV_PROTECT) {
    return addon.kvCompact(ctx, budget, protect);
  }
  // src/engine-a4b.js:620-657: prefill; past `decap` entries one scored
  // probe step on the whole cache, then compaction; budget-maintained decode
  // in chunks of <= 8, recompacting before a chunk would pass `decap`
  async function generateLong(inputIds, maxNew, eosIds = new Set([106, 1]),
                              { budget = KV_BUDGET, protect = KV_PROTECT, decap = KV_DECAP } = {}) {
    const g0 = await prefill(inputIds);
    const out = [g0];
    if (eosIds.has(g0)) return out;
    let pos = inputIds.length, done = 1;
    if (addon.kvCount(ctx) > decap) {
      const t = decodeChunk(pos, 1, 0)[0];
      pos += 1;
      out.push(t);
      done = 2;
      await compactAll(budget, protect);
      if (eosIds.has(t)) return out;
    }
    while (done < maxNew) {
      if (addon.kvCount(ctx) + 8 > decap) await compactAll(budget, protect);
      const n = Math.min(8, maxNew - done);
      const toks = decodeChunk(pos, n, done - 1);
      pos += n;
      let stop = false;
      for (let k = 0; k < n; k++) {
        out.push(toks[k]);
        if (eosIds.has(toks[k])) { stop = true; break; }
      }
      done += n;
      if (stop) break;
    }
    return out.slice(0, maxNew);
  }
  function kvCount() { return addon.kvCount(ctx); }
  async function readHidden() { return addon.readHidden(ctx); }
  async function readLayerHidden(layer) { return addon.readLayerHidden(ctx, layer); }
  async function readLogits() { return addon.readLogits(ctx); }
  function reset() { addon.reset(ctx); }
  function close() { addon.destroy(ctx); }

  return { C, step, argmaxFast, decodeChunk, generateFast, prefill, generatePrefill, profileStep, profilePrefill,
           compactAll, generateLong, kvCount, readHidden, readLayerHidden, readLogits, reset, close, tokRing };
}

module.exports = { loadEngine, configFromKV, addon, FLAG_NO_GRAPH, FLAG_STEP_PREFILL, FLAG_KV_SCORE, FLAG_LAYER_HIDDEN,
                   KV_BUDGET,
                   KV_DECAP, KV_PROTECT };
