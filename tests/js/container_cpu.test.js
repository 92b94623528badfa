// The container from Node without a GPU: reads the header of files tests/test_js_facade.py
// wrote, prints it as one JSON line for the Python side to compare, and checks that a
// malformed file throws EnargeiaError with the reference's message (enargeia.ts:96-110).
//
//   node tests/js/container_cpu.test.js <good.enargeia> <bad-magic.enargeia>
'use strict';

const path = require('path');
const { describe, it, expect, expectThrows, run } = require('./harness.js');
const eg = require(path.join(__dirname, '..', '..', 'enargeia_amd', 'js', 'index.js'));

const [good, bad] = process.argv.slice(2);

describe('container', () => {
  it('reads the header and the tensor table', () => {
    const h = eg.readEnargeiaHeader(good);
    expect(h.version === eg.ENARGEIA_VERSION && h.tensors instanceof Map, 'EnargeiaHeader shape');
    const out = { blockSize: h.blockSize, quantization: h.quantization, dataOffset: h.dataOffset,
      fileSize: h.fileSize, tensors: {} };
    for (const [name, t] of h.tensors) out.tensors[name] = t;
    process.stdout.write('HEADER ' + JSON.stringify(out) + '\n');
  });

  it('throws EnargeiaError for a foreign file', () => {
    expectThrows(() => eg.readEnargeiaHeader(bad), (e) => {
      expect(e instanceof eg.EnargeiaError && e.name === 'EnargeiaError', `${e.name}`);
      expect(e.message === 'not a .enargeia file: magic is "SAFETENS"', e.message);
    }, 'bad magic');
  });
});

run();
