// gguf.js -- GGUF v2/v3 reader for the Node host: openGGUF(path) parses the
// header, key/value metadata and tensor table once and returns
// { kv, tensors, dataStart, fetch(name) }, fetch giving { name, dims, type,
// offset, buf } with only that tensor's bytes read from the file -- the
// interface of openGGUF (src/gguf.js:17-83), which does the same over HTTP
// byte ranges.  tokenizer.* arrays are dropped, as there.
"use strict";
const fs = require("fs");

const GGML = { F32: 0, F16: 1, Q4_0: 2, Q5_0: 6, Q8_0: 8, Q4_K: 12, Q6_K: 14, BF16: 30 };
const TYPE_SIZES = {  // [blockBytes, blockElems]
  [GGML.F32]: [4, 1], [GGML.F16]: [2, 1], [GGML.BF16]: [2, 1],
  [GGML.Q4_0]: [18, 32], [GGML.Q5_0]: [22, 32], [GGML.Q8_0]: [34, 32],
  [GGML.Q4_K]: [144, 256], [GGML.Q6_K]: [210, 256],
};

function tensorBytes(t) {
  const ts = TYPE_SIZES[t.type];
  if (!ts) throw new Error(`unknown ggml type ${t.type}`);
  const n = t.dims.reduce((a, b) => a * b, 1);
  if (n % ts[1]) throw new Error(`${t.name}: ${n} elements are not whole blocks of ${ts[1]}`);
  return (n / ts[1]) * ts[0];
}

// header reader over a growing prefix of the file
function reader(fd, size) {
  let buf = Buffer.alloc(0);
  let off = 0;
  function need(n) {
    if (off + n <= buf.length) return;
    if (off + n > size) throw new Error("truncated GGUF header");
    const want = Math.min(size, Math.max(off + n, 2 * buf.length, 1 << 20));
    const nb = Buffer.alloc(want);
    buf.copy(nb, 0, 0, buf.length);
    fs.readSync(fd, nb, buf.length, want - buf.length, buf.length);
    buf = nb;
  }
  const r = {
    get off() { return off; },
    u8() { need(1); return buf.readUInt8(off++); },
    u32() { need(4); const v = buf.readUInt32LE(off); off += 4; return v; },
    u64() {
      need(8);
      const v = buf.readBigUInt64LE(off);
      off += 8;
      if (v > BigInt(Number.MAX_SAFE_INTEGER)) throw new Error("GGUF value beyond 2^53");
      return Number(v);
    },
    str() { const n = r.u64(); need(n); const s = buf.toString("utf8", off, off + n); off += n; return s; },
    scalar(t) {
      switch (t) {
        case 0: return r.u8();
        case 1: { need(1); const v = buf.readInt8(off); off += 1; return v; }
        case 2: { need(2); const v = buf.readUInt16LE(off); off += 2; return v; }
        case 3: { need(2); const v = buf.readInt16LE(off); off += 2; return v; }
        case 4: return r.u32();
        case 5: { need(4); const v = buf.readInt32LE(off); off += 4; return v; }
        case 6: { need(4); const v = buf.readFloatLE(off); off += 4; return v; }
        case 7: return r.u8() !== 0;
        case 10: return r.u64();
        case 11: { need(8); const v = Number(buf.readBigInt64LE(off)); off += 8; return v; }
        case 12: { need(8); const v = buf.readDoubleLE(off); off += 8; return v; }
        default: throw new Error(`unknown GGUF value type ${t}`);
      }
    },
  };
  return r;
}

function openGGUF(path) {
  const fd = fs.openSync(path, "r");
  const size = fs.fstatSync(fd).size;
  const r = reader(fd, size);
  const magic = Buffer.alloc(4);
  fs.readSync(fd, magic, 0, 4, 0);
  if (magic.toString("latin1") !== "GGUF") {
    fs.closeSync(fd);
    throw new Error("not GGUF");
  }
  for (let i = 0; i < 4; i++) r.u8();
  const version = r.u32();
  if (version !== 2 && version !== 3) throw new Error(`unsupported GGUF version ${version}`);
  const nTensors = r.u64();
  const nKV = r.u64();
  function val(t) {
    if (t === 8) return r.str();
    if (t === 9) {
      const et = r.u32(), n = r.u64();
      const out = [];
      for (let i = 0; i < n; i++) out.push(val(et));
      return out;
    }
    return r.scalar(t);
  }
  const kv = {};
  for (let i = 0; i < nKV; i++) {
    const k = r.str();
    const t = r.u32();
    kv[k] = val(t);
    if (k.startsWith("tokenizer.")) delete kv[k];
  }
  const align = kv["general.alignment"] !== undefined ? kv["general.alignment"] : 32;
  const tensors = {};
  for (let i = 0; i < nTensors; i++) {
    const name = r.str();
    const nd = r.u32();
    const dims = [];
    for (let d = 0; d < nd; d++) dims.push(r.u64());
    const type = r.u32();
    const offset = r.u64();
    tensors[name] = { name, dims, type, offset };
  }
  const dataStart = Math.ceil(r.off / align) * align;
  return {
    kv, tensors, dataStart,
    async fetch(name) {
      const t = tensors[name];
      if (!t) throw new Error("no tensor " + name);
      const n = tensorBytes(t);
      const start = dataStart + t.offset;
      if (start + n > size) throw new Error(`tensor ${name} extends past the end of the file`);
      const buf = Buffer.alloc(n);
      fs.readSync(fd, buf, 0, n, start);
      return Object.assign({}, t, { buf });
    },
    close() { fs.closeSync(fd); },
  };
}

module.exports = { GGML, TYPE_SIZES, tensorBytes, openGGUF };
