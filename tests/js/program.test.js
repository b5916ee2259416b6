'use strict';
// Mirrors the reference's tests/api/program.test.ts.
const W = require('../../wgpu-executorch_amd/js');
const { describe, it, expect, expectTensorClose } = require('./harness');
const { WgpuExecutionContext } = W;
let cached = null;
async function setupGPU() { if (!cached) cached = await W.requestDevice(global.WGX_DEVICE_INDEX); return cached; }

// out = (a + 1.5 * b) @ c, with pool reuse (a and out share pool 0)
const prog = {
  version: '1',
  chain: [
    { name: 'aten.add.Tensor', args: [0, 1, 2, 3] },
    { name: 'aten.mm.default', args: [3, 4, 5] },
  ],
  values: [
    { type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 0 },
    { type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 1 },
    { type: 'scalar', value: 1.5 },
    { type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 2 },
    { type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 3 },
    { type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 0 },
  ],
  inputIds: [0, 1, 4],
  outputIds: [5],
  memoryPlan: { pools: [{ id: 0, size: 16 }, { id: 1, size: 16 }, { id: 2, size: 16 }, { id: 3, size: 16 }] },
};
const weights = new ArrayBuffer(0);
async function inputs(ctx) {
  return [
    ctx.tensor('float32', [2, 2]).setData(new Float32Array([1, 2, 3, 4])),
    ctx.tensor('float32', [2, 2]).setData(new Float32Array([10, 20, 30, 40])),
    ctx.tensor('float32', [2, 2]).setData(new Float32Array([1, 2, 3, 4])),
  ];
}

describe('WgpuExecutionContext.recordProgram()', () => {
  it('runs a 2-kernel program with buffer reuse', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const [a, b, c] = await inputs(ctx);
    const out = ctx.tensor('float32', [2, 2]);
    ctx.recordProgram(prog, weights, [a, b, c, out]);
    ctx.submit();
    await ctx.sync();
    await expectTensorClose(W, out, [112, 160, 240, 352]);
    ctx.submit();  // replay
    await ctx.sync();
    await expectTensorClose(W, out, [112, 160, 240, 352]);
    ctx.destroy();
  }, { gpu: true });
  it('rejects wrong arg count', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const [a, b, c] = await inputs(ctx);
    expect(() => ctx.recordProgram(prog, weights, [a, b, c])).toThrow(/expected 4 args/);
    ctx.destroy();
  });
  it('rejects non-Tensor output', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const [a, b, c] = await inputs(ctx);
    expect(() => ctx.recordProgram(prog, weights, [a, b, c, 42])).toThrow(/output 0 must be a Tensor/);
    ctx.destroy();
  });
  it('rejects unknown operator', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const [a, b, c] = await inputs(ctx);
    const bad = Object.assign({}, prog, { chain: [{ name: 'aten.nonexistent.default', args: [0, 1, 2, 3] }] });
    expect(() => ctx.recordProgram(bad, weights, [a, b, c, ctx.tensor('float32', [2, 2])])).toThrow(/unknown operator/);
    ctx.destroy();
  });
  it('rejects missing memory pool', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const [a, b, c] = await inputs(ctx);
    const bad = Object.assign({}, prog, {
      values: [{ type: 'tensor', shape: [2, 2], dtype: 'float32', memObjId: 99 }].concat(prog.values.slice(1)),
    });
    expect(() => ctx.recordProgram(bad, weights, [a, b, c, ctx.tensor('float32', [2, 2])])).toThrow(/no memory pool 99/);
    ctx.destroy();
  });
  it('resolveArgs maps tensors, scalars, lists, tensor lists and nulls', async () => {
    const tensors = new Map([[0, 'T0'], [3, 'T3']]);
    const values = [{ type: 'tensor' }, { type: 'scalar', value: 2 }, { type: 'list', items: [1, 2] },
      { type: 'tensor' }, { type: 'tensorlist', items: [0, 3] }, { type: 'null' }];
    const r = W.resolveArgs({ name: 'x', args: [0, 1, 2, 4, 5] }, values, tensors);
    expect(r).toEqual(['T0', 2, [1, 2], ['T0', 'T3'], undefined]);
    expect(() => W.resolveArgs({ name: 'y', args: [4] }, [{ type: 'tensor' }, { type: 'scalar', value: 1 },
      { type: 'tensor' }, { type: 'tensor' }, { type: 'tensorlist', items: [1] }], tensors)).toThrow(/tensorlist item 1 is not a tensor/);
  });
});

// ------------------------------------------------------------ zero-copy cat / split / view_copy
const T = (shape, extra) => Object.assign({ type: 'tensor', shape, dtype: 'float32' }, extra || {});
const L = (items) => ({ type: 'list', items });
const S = (value) => ({ type: 'scalar', value });
const TL = (items) => ({ type: 'tensorlist', items });
const add = (a, b, alpha, out) => ({ name: 'aten.add.Tensor', args: [a, b, alpha, out] });
const cat = (list, dim, out) => ({ name: 'aten.cat.default', args: [list, dim, out] });
const split = (x, sizes, dim, outs) => ({ name: 'aten.split_with_sizes_copy.default', args: [x, sizes, dim, outs] });
const elidedOf = (p) => [...W._planViews(p).elided].sort((a, b) => a - b);

// x [1,4,2,2] -> t = x + x -> split [p(1ch), q(3ch)] -> r = q + q ->
// y = cat[r, p] (dim 1) and z = cat[p, r] (p, r in two cats: one copies) ->
// out = y + z
function viewProgram() {
  return {
    version: '1',
    chain: [
      add(0, 0, 1, 2),
      split(2, 3, 4, 5),
      add(7, 7, 1, 8),
      cat(9, 1, 10),
      cat(11, 1, 12),
      add(10, 12, 1, 13),
    ],
    values: [
      T([1, 4, 2, 2], { memObjId: 0 }), S(1), T([1, 4, 2, 2], { memObjId: 1 }),
      L([1, 3]), S(1), TL([6, 7]), T([1, 1, 2, 2], { memObjId: 2 }), T([1, 3, 2, 2], { memObjId: 3 }),
      T([1, 3, 2, 2], { memObjId: 1 }), TL([8, 6]), T([1, 4, 2, 2], { memObjId: 0 }),
      TL([6, 8]), T([1, 4, 2, 2], { memObjId: 4 }), T([1, 4, 2, 2], { memObjId: 5 }),
    ],
    inputIds: [0],
    outputIds: [13],
    memoryPlan: { pools: [0, 1, 2, 3, 4, 5].map((id) => ({ id, size: 64 })) },
  };
}

describe('recordProgram views', () => {
  it('ties a split and the first cat; the second cat of the same pieces copies', () => {
    const p = viewProgram();
    expect(elidedOf(p)).toEqual([1, 3]);
    const plan = W._planViews(p);
    // y = [r | p], t = [p | q]: r and q share no bytes with p in either
    const at = (id) => plan.place.get(id).off;
    expect(at(8) - at(10)).toEqual(0);
    expect(at(6) - at(10)).toEqual(48);
    expect(at(6) - at(2)).toEqual(0);
    expect(at(7) - at(2)).toEqual(16);
    expect(plan.place.has(0) || plan.place.has(13)).toBe(false);
  });
  it('rejects a cat that repeats a piece, outputs, inputs and non-leading dimensions', () => {
    const rep = viewProgram();
    rep.chain = [add(0, 0, 1, 6), { name: 'aten.cat.default', args: [5, 4, 13] }, add(13, 13, 1, 12)];
    rep.values[5] = TL([6, 6]);
    rep.values[6] = T([1, 2, 2, 2], { memObjId: 2 });
    rep.outputIds = [12];
    expect(elidedOf(rep)).toEqual([]);
    rep.values[5] = TL([6, 3]);
    rep.values[3] = T([1, 2, 2, 2]);
    rep.chain.splice(1, 0, add(0, 0, 1, 3));
    expect(elidedOf(rep)).toEqual([2]);
    const out = viewProgram();
    out.outputIds = [10];
    expect(elidedOf(out)).toEqual([1]);
    const inp = { version: '1', chain: [add(4, 4, 2, 5), cat(1, 2, 3), add(3, 3, 2, 6)],
      values: [T([1, 2, 2, 2]), TL([0, 5]), S(1), T([1, 4, 2, 2]), T([1, 2, 2, 2]), T([1, 2, 2, 2]), T([1, 4, 2, 2])],
      inputIds: [0, 4], outputIds: [6], memoryPlan: { pools: [] } };
    expect(elidedOf(inp)).toEqual([]);
    inp.chain.unshift(add(4, 4, 2, 0));
    inp.inputIds = [4];
    expect(elidedOf(inp)).toEqual([2]);
    const deep = { version: '1',
      chain: [add(0, 0, 1, 2), add(0, 0, 1, 3), cat(4, 5, 6), add(6, 6, 1, 7)],
      values: [T([1, 2, 3]), S(1), T([1, 2, 3]), T([1, 2, 3]), TL([2, 3]), S(2), T([1, 2, 6]), T([1, 2, 6])],
      inputIds: [0], outputIds: [7], memoryPlan: { pools: [] } };
    expect(elidedOf(deep)).toEqual([]);
    deep.values[5] = S(1);
    deep.values[6] = T([1, 4, 3]);
    deep.values[7] = T([1, 4, 3]);
    expect(elidedOf(deep)).toEqual([2]);
    deep.values[5] = S(-2);
    expect(elidedOf(deep)).toEqual([2]);
  });
  it('ties flat copies: clone without a memory format, squeeze_copy, unsqueeze_copy', () => {
    // t = x + x -> c = clone(t) -> s = squeeze_copy(c, [0]) -> u = unsqueeze_copy(s, 0)
    // -> out = u + u; then the same with a memory format on the clone
    const flat = (memfmt) => ({
      version: '1',
      chain: [
        add(0, 0, 1, 2),
        { name: 'aten.clone.default', args: [2, 3, 4] },
        { name: 'aten.squeeze_copy.dims', args: [4, 5, 6] },
        { name: 'aten.unsqueeze_copy.default', args: [6, 7, 8] },
        add(8, 8, 1, 9),
      ],
      values: [
        T([1, 4, 2, 2], { memObjId: 0 }), S(1), T([1, 4, 2, 2], { memObjId: 1 }),
        memfmt ? S(memfmt) : { type: 'null' }, T([1, 4, 2, 2], { memObjId: 2 }),
        L([0]), T([4, 2, 2], { memObjId: 1 }), S(0), T([1, 4, 2, 2], { memObjId: 2 }),
        T([1, 4, 2, 2], { memObjId: 3 }),
      ],
      inputIds: [0],
      outputIds: [9],
      memoryPlan: { pools: [0, 1, 2, 3].map((id) => ({ id, size: 64 })) },
    });
    const p = flat(null);
    expect(elidedOf(p)).toEqual([1, 2, 3]);
    const plan = W._planViews(p);
    for (const id of [4, 6, 8]) expect(plan.place.get(id).off - plan.place.get(2).off).toEqual(0);
    expect(elidedOf(flat(2))).toEqual([2, 3]);
  });
  // o1 = a + b, o2 = a * b, o3 = o1 + o2, all three program outputs
  const threeOut = () => ({
    version: '1',
    chain: [
      { name: 'aten.add.Tensor', args: [0, 1, 2, 3] },
      { name: 'aten.mul.Tensor', args: [0, 1, 4] },
      { name: 'aten.add.Tensor', args: [3, 4, 2, 5] },
    ],
    values: [
      { type: 'tensor', shape: [4], dtype: 'float32', memObjId: 0 },
      { type: 'tensor', shape: [4], dtype: 'float32', memObjId: 1 },
      { type: 'scalar', value: 1 },
      { type: 'tensor', shape: [4], dtype: 'float32', memObjId: 2 },
      { type: 'tensor', shape: [4], dtype: 'float32', memObjId: 3 },
      { type: 'tensor', shape: [4], dtype: 'float32', memObjId: 4 },
    ],
    inputIds: [0, 1],
    outputIds: [3, 4, 5],
    memoryPlan: { pools: [0, 1, 2, 3, 4].map((id) => ({ id, size: 16 })) },
  });
  it('binds no tensor when two program outputs share memory', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const a = ctx.tensor('float32', [4]).setData(new Float32Array([1, 2, 3, 4]));
    const b = ctx.tensor('float32', [4]).setData(new Float32Array([5, 6, 7, 8]));
    const t = ctx.tensor('float32', [4]);
    const u = ctx.tensor('float32', [4]);
    ctx.recordProgram(threeOut(), weights, [a, b, t, t, u]);
    // 3 ops, 2 input copies, 3 output copies: nothing is bound
    expect(ctx.commandCount).toBe(8);
    const ok = new WgpuExecutionContext(await setupGPU());
    ok.recordProgram(threeOut(), weights, [a, b, ok.tensor('float32', [4]), ok.tensor('float32', [4]), ok.tensor('float32', [4])]);
    expect(ok.commandCount).toBe(3);  // disjoint outputs: every input and output bound
    ok.destroy();
    if (ctx.device.index >= 0) {
      ctx.submit();
      await ctx.sync();
      await expectTensorClose(W, t, [5, 12, 21, 32]);  // the later copy (o2) wins
      await expectTensorClose(W, u, [11, 20, 31, 44]);
    }
    ctx.destroy();
  });
  it('runs split/cat chains with and without views', async () => {
    const x = new Float32Array(16).map((_, i) => i - 5.5);
    const t = x.map((v) => 2 * v);
    const p = t.slice(0, 4), q = t.slice(4);
    const r = q.map((v) => 2 * v);
    const y = [...r, ...p], z = [...p, ...r];
    const want = y.map((v, i) => v + z[i]);
    for (const views of [true, false]) {
      const ctx = new WgpuExecutionContext(await setupGPU());
      const xin = ctx.tensor('float32', [1, 4, 2, 2]).setData(x);
      const out = ctx.tensor('float32', [1, 4, 2, 2]);
      ctx.recordProgram(viewProgram(), weights, [xin, out], { views });
      for (let rep = 0; rep < 2; rep++) {
        ctx.submit();
        await ctx.sync();
        await expectTensorClose(W, out, want);
      }
      ctx.destroy();
    }
  }, { gpu: true });
});
