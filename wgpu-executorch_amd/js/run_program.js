'use strict';
/**
 * Records a program.json + weights.bin with WgpuExecutionContext.recordProgram
 * (src/context.ts:219-317) and runs it on one GPU.
 *
 *   node run_program.js DIR [--device N] [--warmup W] [--reps R] [--out FILE] [--record-only]
 *
 * DIR holds program.json, weights.bin and input.bin (the program's single
 * input, raw element bytes of its dtype).  The program is recorded once and
 * every frame is one submit() + sync(), the reference's serving loop
 * (example/src/tasks/yolo26-detection/loop.ts:141-189).  Prints one JSON line:
 *   frame_ms_wall    median wall time of submit()+sync() per frame
 *   frame_ms_device  mean device time per submit over R back-to-back submits
 *                    (HIP events on the queue)
 * and, with --out, writes the output tensor's bytes after the timed frames.
 * --record-only validates and records the program without running it (it
 * works on the host-only device -1).  --no-fuse records no conv -> sigmoid ->
 * mul folding, --no-views runs every cat / split / view_copy as a copy,
 * --no-bind-io copies the input into and the output out of the memory plan
 * instead of binding the caller's tensors,
 * --eager replays the recorded launches one by one on the stream instead of
 * through a HIP graph.  The program is checked with the converter's rules
 * (validateProgram) before it is recorded.
 */
const fs = require('fs');
const path = require('path');
const W = require('./index.js');

function parseArgs(argv) {
  const a = { dir: null, device: 0, warmup: 5, reps: 50, out: null, recordOnly: false, fuse: true, views: true,
    bindIO: true, eager: false };
  for (let i = 0; i < argv.length; i++) {
    const k = argv[i];
    if (k === '--device') a.device = Number(argv[++i]);
    else if (k === '--warmup') a.warmup = Number(argv[++i]);
    else if (k === '--reps') a.reps = Number(argv[++i]);
    else if (k === '--out') a.out = argv[++i];
    else if (k === '--record-only') a.recordOnly = true;
    else if (k === '--no-fuse') a.fuse = false;
    else if (k === '--no-views') a.views = false;
    else if (k === '--no-bind-io') a.bindIO = false;
    else if (k === '--eager') a.eager = true;
    else a.dir = k;
  }
  if (!a.dir) throw new Error('usage: node run_program.js DIR [--device N] [--warmup W] [--reps R] [--out FILE]');
  return a;
}

async function main() {
  const args = parseArgs(process.argv.slice(2));
  const program = JSON.parse(fs.readFileSync(path.join(args.dir, 'program.json'), 'utf8'));
  const wbuf = fs.readFileSync(path.join(args.dir, 'weights.bin'));
  const weights = wbuf.buffer.slice(wbuf.byteOffset, wbuf.byteOffset + wbuf.byteLength);
  const ibuf = fs.readFileSync(path.join(args.dir, 'input.bin'));

  W.validateProgram(program, weights.byteLength);
  const device = await W.requestDevice(args.device);
  const ctx = new W.WgpuExecutionContext(device);
  const inV = program.values[program.inputIds[0]];
  const outV = program.values[program.outputIds[0]];
  const input = ctx.tensor(inV.dtype, inV.shape);
  input.setData(new Uint8Array(ibuf.buffer, ibuf.byteOffset, ibuf.byteLength));
  const output = ctx.tensor(outV.dtype, outV.shape);

  if (args.eager) ctx.setGraphMode(false);
  const t0 = process.hrtime.bigint();
  ctx.recordProgram(program, weights, [input, output], { fuse: args.fuse, views: args.views, bindIO: args.bindIO });
  const recordMs = Number(process.hrtime.bigint() - t0) / 1e6;
  if (args.recordOnly) {
    console.log(JSON.stringify({ record_ms: recordMs, commands: ctx.commandCount, ops: program.chain.length }));
    ctx.destroy();
    device.destroy();
    return;
  }

  for (let i = 0; i < args.warmup; i++) { ctx.submit(); await ctx.sync(); }
  const samples = [];
  for (let i = 0; i < args.reps; i++) {
    const s = process.hrtime.bigint();
    ctx.submit();
    await ctx.sync();
    samples.push(Number(process.hrtime.bigint() - s) / 1e6);
  }
  samples.sort((x, y) => x - y);
  const deviceMs = ctx.timeSubmits(args.reps);
  if (args.out) {
    const data = await output.getData();
    fs.writeFileSync(args.out, Buffer.from(data));
  }
  console.log(JSON.stringify({
    frame_ms_wall: samples[Math.floor(samples.length / 2)],
    frame_ms_wall_min: samples[0],
    frame_ms_device: deviceMs,
    record_ms: recordMs,
    commands: ctx.commandCount,
    ops: program.chain.length,
  }));
  ctx.destroy();
  device.destroy();
}

main().catch((e) => { console.error(e && e.stack ? e.stack : String(e)); process.exit(1); });
