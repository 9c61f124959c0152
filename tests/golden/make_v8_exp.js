// Writes Math.exp(x) for a fixed set of inputs, as little-endian f64 bytes,
// to pin the oracle's and the GPU's exp (fdlibm algorithm) to the JS
// engine's results.  Usage: node tests/golden/make_v8_exp.js > tests/golden/v8_exp.json
'use strict';
const buf = new DataView(new ArrayBuffer(8));
function bits(x) { buf.setFloat64(0, x); return buf.getBigUint64(0); }
function fromBits(b) { buf.setBigUint64(0, b); return buf.getFloat64(0); }
let s = 0x6A09E667;
function rnd() { s = (Math.imul(s, 1664525) + 1013904223) >>> 0; return s; }
const inputs = [];
// the sampling softmax domain: (v - max) / temperature <= 0, f32 logits widened
for (let i = 0; i < 14000; i++) {
  const a = Math.fround((rnd() / 4294967296) * 60 - 30);
  const b = Math.fround((rnd() / 4294967296) * 60 - 30);
  const temps = [1, 0.7, 0.5, 1.3, 2, 0.1];
  inputs.push((Math.min(a, b) - Math.max(a, b)) / temps[i % temps.length]);
}
// the whole finite range, uniform in the exponent
for (let i = 0; i < 8000; i++) {
  const e = (rnd() % 20) - 10;
  const m = rnd() / 4294967296;
  let x = (1 + m) * Math.pow(2, e);
  if (rnd() & 1) x = -x;
  inputs.push(x);
}
for (let i = 0; i < 1000; i++) inputs.push((rnd() / 4294967296) * 1454 - 745);
// thresholds: 2^-28, 0.5 ln2, 1.5 ln2, over/underflow limits, subnormal results, 1
const edges = [Math.pow(2, -28), 0.5 * Math.LN2, 1.5 * Math.LN2, 709.782712893384, 745.1332191019411,
  708.3964185322641, 1, 0.5, 2, 10, 100, 700, 730];
for (const t of edges) for (let d = -3n; d <= 3n; d++) {
  const y = fromBits(bits(t) + d);
  inputs.push(y, -y);
}
inputs.push(0, -0, 1, -1, 1e-300, -1e-300, 1e-320, Infinity, -Infinity, NaN, -1022 * Math.LN2, -1074 * Math.LN2);
const xs = Float64Array.from(inputs);
const ys = xs.map((x) => Math.exp(x));
process.stdout.write(JSON.stringify({
  engine: 'node ' + process.version,
  count: xs.length,
  x_f64le_base64: Buffer.from(xs.buffer).toString('base64'),
  exp_f64le_base64: Buffer.from(ys.buffer).toString('base64'),
}) + '\n');
