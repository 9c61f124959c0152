// Writes the JS engine's RoPE primitives for a set of decode positions:
// thetaScale = Math.pow(base, -2 / nDims), the angles theta_0 = position,
// theta_{i+1} = Math.fround(theta_i * thetaScale), and Math.cos / Math.sin of
// each angle, as little-endian f64 bytes.  They pin the oracle's pow, angle
// recurrence and trigonometry (glibc's) to the engine's (fdlibm's).
// Usage: node tests/golden/make_v8_rope.js > tests/golden/v8_rope.json
'use strict';
const positions = [0, 1, 2, 3, 17, 100, 511, 4095, 4096, 32767, 131071];
const cases = [];
for (const base of [10000, 1000000]) {
  for (const nDims of [256, 128]) {
    const scale = Math.pow(base, -2 / nDims);
    for (const position of positions) {
      const thetas = [];
      let theta = position;
      for (let i = 0; i < nDims / 2; i++) {
        thetas.push(theta);
        theta = Math.fround(theta * scale);
      }
      const t = Float64Array.from(thetas);
      cases.push({
        base, nDims, position, scale,
        theta_f64le_base64: Buffer.from(t.buffer).toString('base64'),
        cos_f64le_base64: Buffer.from(t.map(Math.cos).buffer).toString('base64'),
        sin_f64le_base64: Buffer.from(t.map(Math.sin).buffer).toString('base64'),
      });
    }
  }
}
process.stdout.write(JSON.stringify({ engine: 'node ' + process.version, cases }) + '\n');
