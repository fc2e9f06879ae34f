// run_greedy.js -- command-line driver of the JS host:
//   node run_greedy.js <model.gguf> <id,id,...> <maxNew> ['{"ring":16,...}'] ['{"budget":16,...}']
// loads the model through engine.js, runs generateFast (batched prefill then
// GPU-fed decode), then the step API on the same prompt after a reset, and
// prints one JSON line: {generate, steps, hidden_l2, logits_max}; with the
// fifth argument (generateLong options; the model needs flags FLAG_KV_SCORE)
// also generate_long and kv_count after a generateLong of maxNew tokens.
"use strict";
const { loadEngine } = require("./engine");

async function main() {
  const [file, idsArg, maxNewArg, ovArg, longArg] = process.argv.slice(2);
  if (!file || !idsArg || !maxNewArg) {
    console.error("usage: node run_greedy.js model.gguf id,id,... maxNew [overrides-json]");
    process.exit(2);
  }
  const ids = idsArg.split(",").map(Number);
  const maxNew = Number(maxNewArg);
  const eng = await loadEngine(file, ovArg ? JSON.parse(ovArg) : {});
  const generate = await eng.generateFast(ids, maxNew, new Set());
  eng.reset();
  const steps = [];
  let pos = 0;
  for (const t of ids) steps.push(await eng.step(t, pos++));
  const hidden = await eng.readHidden();
  const logits = await eng.readLogits();
  let l2 = 0, lmax = -Infinity;
  for (const v of hidden) l2 += v * v;
  for (const v of logits) lmax = Math.max(lmax, v);
  const res = { generate, steps, hidden_l2: Math.sqrt(l2), logits_max: lmax };
  if (longArg) {
    eng.reset();
    res.generate_long = await eng.generateLong(ids, maxNew, new Set(), JSON.parse(longArg));
    res.kv_count = eng.kvCount();
  }
  eng.close();
  console.log(JSON.stringify(res));
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : String(e));
  process.exit(1);
});
