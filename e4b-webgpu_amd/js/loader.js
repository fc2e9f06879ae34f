// loader.js -- safetensors reader for the Node host, the interface of
// src/loader.js: openSafetensors(path) reads the u64 header length and the
// JSON index once (dropping __metadata__) and returns { path, index, has,
// info, fetch(name) }, fetch giving the index entry plus buf, that tensor's
// bytes only (one file read per tensor, where the reference issues one HTTP
// byte range); bf16ToF32 widens bf16 bits to f32 by a 16-bit shift;
// f32Scalar reads the first f32 of a buffer (0 when empty).
"use strict";
const fs = require("fs");

function openSafetensors(file) {
  const fd = fs.openSync(file, "r");
  const size = fs.fstatSync(fd).size;
  const head = Buffer.alloc(8);
  if (size < 8 || fs.readSync(fd, head, 0, 8, 0) !== 8) {
    fs.closeSync(fd);
    throw new Error(`${file}: shorter than the 8-byte header length`);
  }
  const n = Number(head.readBigUInt64LE(0));
  if (8 + n > size) {
    fs.closeSync(fd);
    throw new Error(`${file}: header of ${n} bytes extends past the end of the file`);
  }
  const hj = Buffer.alloc(n);
  fs.readSync(fd, hj, 0, n, 8);
  const index = JSON.parse(hj.toString("utf8"));
  delete index.__metadata__;
  const base = 8 + n;
  return {
    path: file,
    index,
    has: (name) => name in index,
    info: (name) => index[name],
    async fetch(name) {
      const t = index[name];
      if (!t) throw new Error(`tensor not found: ${name}`);
      const [a, b] = t.data_offsets;
      const buf = Buffer.alloc(b - a);
      if (b > a) fs.readSync(fd, buf, 0, b - a, base + a);
      return Object.assign({}, t, { buf: buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.length) });
    },
    close: () => fs.closeSync(fd),
  };
}

function bf16ToF32(buf) {
  const u16 = new Uint16Array(buf);
  const out = new Float32Array(u16.length);
  const u32 = new Uint32Array(out.buffer);
  for (let i = 0; i < u16.length; i++) u32[i] = u16[i] << 16;
  return out;
}

function f32Scalar(buf) {
  const f = new Float32Array(buf);
  return f.length ? f[0] : 0;
}

module.exports = { openSafetensors, bf16ToF32, f32Scalar };
