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
