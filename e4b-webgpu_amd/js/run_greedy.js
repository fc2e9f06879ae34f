// run_greedy.js -- command-line driver of the JS host:
//   node run_greedy.js <model.gguf> <id,id,...> <maxNew> ['{"ring":16,...}'] ['{"budget":16,...}']
// loads the model through engine.js, runs generateFast (the prompt through
// the step, then GPU-fed decode; with E4B_LOGITS_OUT set its last logits go
// to that file as raw f32), generatePrefill (batched prefill, same decode),
// profilePrefill, then the step API on the same prompt after a reset and one
// profileStep, and prints one JSON line: {generate, generate_prefill, steps,
// hidden_l2, logits_max, profile_step, profile_prefill}; with the
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
  const logitsOut = process.env.E4B_LOGITS_OUT;  // the last step's logits of generateFast, raw f32
  if (logitsOut) require("fs").writeFileSync(logitsOut, Buffer.from((await eng.readLogits()).buffer));
  eng.reset();
  const generatePrefill = await eng.generatePrefill(ids, maxNew, new Set());
  eng.reset();
  const profPrefill = await eng.profilePrefill(ids);
  eng.reset();
  const steps = [];
  let pos = 0;
  for (const t of ids) steps.push(await eng.step(t, pos++));
  const hidden = await eng.readHidden();
  const logits = await eng.readLogits();
  let l2 = 0, lmax = -Infinity;
  for (const v of hidden) l2 += v * v;
  for (const v of logits) lmax = Math.max(lmax, v);
  const profStep = await eng.profileStep(ids[0], pos);
  const roles = (m) => Array.from(m.entries()).map(([k, v]) => [k, v.n, v.us > 0]);
  const res = { generate, generate_prefill: generatePrefill, steps, hidden_l2: Math.sqrt(l2), logits_max: lmax,
                profile_step: roles(profStep), profile_prefill: roles(profPrefill) };
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
