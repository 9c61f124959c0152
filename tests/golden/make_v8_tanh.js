// Writes Math.tanh(x) for a fixed set of inputs, as little-endian f64 bytes,
// to pin the oracle's tanh (fdlibm algorithm) to the JS engine's results.
// Usage: node tests/golden/make_v8_tanh.js > tests/golden/v8_tanh.json
'use strict';
const buf = new DataView(new ArrayBuffer(8));
function bits(x) { buf.setFloat64(0, x); return buf.getBigUint64(0).toString(16).padStart(16, '0'); }
function fromBits(h) { buf.setBigUint64(0, BigInt('0x' + h)); return buf.getFloat64(0); }
// deterministic LCG over 32-bit words
let s = 0x2545F491;
function rnd() { s = (Math.imul(s, 1664525) + 1013904223) >>> 0; return s; }
const inputs = [];
// the gelu/softcap domain: f32 values in [-48, 48], uniform in bits within ranges
for (let i = 0; i < 40000; i++) {
  const e = (rnd() % 40) - 34;              // magnitude 2^-34 .. 2^5
  const m = rnd() / 4294967296;
  let x = Math.fround((1 + m) * Math.pow(2, e));
  if (rnd() & 1) x = -x;
  inputs.push(x);
}
// thresholds of the algorithm: 2^-28, 0.5 ln2, 1.5 ln2, 1, 22 and neighbours
const edges = [Math.pow(2, -28), 0.5 * Math.LN2, 1.5 * Math.LN2, 1, 22, 0.25, 0.5, 3, 10, 20];
for (const t of edges) for (const d of [-2, -1, 0, 1, 2]) {
  const x = fromBits(bits(t).replace(/.{4}$/, '0000'));
  const y = x + d * Math.pow(2, Math.floor(Math.log2(x)) - 52);
  inputs.push(y, -y);
}
inputs.push(0, -0, 1e-300, -1e-300, 30, -30, 100);
const xs = Float64Array.from(inputs);
const ys = xs.map((x) => Math.tanh(x));
process.stdout.write(JSON.stringify({
  engine: 'node ' + process.version,
  count: xs.length,
  x_f64le_base64: Buffer.from(xs.buffer).toString('base64'),
  tanh_f64le_base64: Buffer.from(ys.buffer).toString('base64'),
}) + '\n');
