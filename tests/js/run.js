'use strict';
// node tests/js/run.js --cpu   : validation/API tests on a host-only device
// node tests/js/run.js --gpu   : every test on GPU 0 (parity KATs included)
const path = require('path');
const H = require('./harness');
const gpu = process.argv.includes('--gpu');
global.WGX_DEVICE_INDEX = gpu ? 0 : -1;
for (const f of ['api.test.js', 'shaders.test.js', 'ops.test.js', 'program.test.js']) require(path.join(__dirname, f));
(async () => {
  let pass = 0; let fail = 0; let skip = 0;
  for (const t of H.tests) {
    if (t.gpu && !gpu) { skip++; continue; }
    try {
      await t.fn();
      pass++;
      console.log(`ok   ${t.name}`);
    } catch (err) {
      fail++;
      console.log(`FAIL ${t.name}: ${err && err.stack ? err.stack.split('\n').slice(0, 3).join(' | ') : err}`);
    }
  }
  console.log(`${pass} passed, ${fail} failed, ${skip} skipped`);
  process.exit(fail ? 1 : 0);
})();
