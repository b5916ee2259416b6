'use strict';
// Minimal describe/it/expect harness (the reference uses vitest, which is not
// installed here).  Tests register with describe/it; run.js executes them.
const tests = [];
let prefix = '';
function describe(name, fn) { const old = prefix; prefix = prefix + name + ' > '; fn(); prefix = old; }
function it(name, fn, opts) { tests.push({ name: prefix + name, fn, gpu: !!(opts && opts.gpu) }); }
function fmt(v) { try { return JSON.stringify(v); } catch (e) { return String(v); } }
function expect(actual) {
  const m = {
    toBe(e) { if (actual !== e) throw new Error(`expected ${fmt(actual)} to be ${fmt(e)}`); },
    toEqual(e) { if (fmt(actual) !== fmt(e)) throw new Error(`expected ${fmt(actual)} to equal ${fmt(e)}`); },
    toBeTruthy() { if (!actual) throw new Error(`expected ${fmt(actual)} to be truthy`); },
    toBeGreaterThanOrEqual(e) { if (!(actual >= e)) throw new Error(`expected ${actual} >= ${e}`); },
    toBeLessThan(e) { if (!(actual < e)) throw new Error(`expected ${actual} < ${e}`); },
    toBeCloseTo(e, digits) {
      const d = digits === undefined ? 2 : digits;
      if (!(Math.abs(actual - e) < Math.pow(10, -d) / 2)) throw new Error(`expected ${actual} to be close to ${e} (${d} digits)`);
    },
    toThrow(re) {
      let threw = null;
      try { actual(); } catch (err) { threw = err; }
      if (!threw) throw new Error('expected function to throw');
      if (re && !re.test(threw.message)) throw new Error(`error "${threw.message}" does not match ${re}`);
    },
  };
  m.not = {
    toThrow() { try { actual(); } catch (err) { throw new Error(`expected no throw, got "${err.message}"`); } },
  };
  m.rejects = {
    async toThrow(re) {
      let threw = null;
      try { await actual; } catch (err) { threw = err; }
      if (!threw) throw new Error('expected promise to reject');
      if (re && !re.test(threw.message)) throw new Error(`rejection "${threw.message}" does not match ${re}`);
    },
  };
  m.resolves = {
    async toBeUndefined() { const v = await actual; if (v !== undefined) throw new Error(`expected undefined, got ${fmt(v)}`); },
  };
  return m;
}
// tests/helpers/assert.ts:10-45 of the reference: max-abs comparison, non-finite rejected
async function expectTensorClose(W, tensor, expected, tolerance) {
  const tol = tolerance === undefined ? 1e-5 : tolerance;
  const data = await tensor.getData();
  const actual = tensor.dtype === 'float16' ? W.fromFloat16Array(data) : new Float32Array(data);
  if (actual.length !== expected.length) throw new Error(`Tensor length mismatch: got ${actual.length}, expected ${expected.length}`);
  let maxDiff = 0; let maxIdx = 0;
  for (let i = 0; i < actual.length; i++) {
    if (!Number.isFinite(actual[i]) || !Number.isFinite(expected[i])) {
      throw new Error(`Non-finite tensor value at index ${i}: got ${actual[i]}, expected ${expected[i]}`);
    }
    const diff = Math.abs(actual[i] - expected[i]);
    if (diff > maxDiff) { maxDiff = diff; maxIdx = i; }
  }
  if (maxDiff > tol) {
    throw new Error(`Tensor mismatch at index ${maxIdx}: got ${actual[maxIdx]}, expected ${expected[maxIdx]} (max diff ${maxDiff.toExponential(3)}, tolerance ${tol})`);
  }
}
module.exports = { tests, describe, it, expect, expectTensorClose };
