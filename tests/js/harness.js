// A minimal describe/it runner for the Node tests (no test framework is installed): runs the
// cases in order, prints one line per case, exits non-zero when any failed. Each case's name
// is printed before it runs, so a run that dies names the case it died in.
'use strict';

const cases = [];
let prefix = '';

function describe(name, body) {
  const saved = prefix;
  prefix = prefix ? `${prefix} > ${name}` : name;
  body();
  prefix = saved;
}

function it(name, fn) {
  cases.push({ name: prefix ? `${prefix} > ${name}` : name, fn });
}

const afterAllHooks = [];
function afterAll(fn) {
  afterAllHooks.push(fn);
}

class AssertionError extends Error {}

function expect(cond, message) {
  if (!cond) throw new AssertionError(message || 'expectation failed');
}

function expectThrows(fn, check, label) {
  let caught = null;
  try {
    fn();
  } catch (err) {
    caught = err;
  }
  expect(caught !== null, `${label}: expected a throw`);
  check(caught);
}

/** compareArrays (test/reference/matmul.ts:56-81): per element |a-e| <= abs + rel*|e|. */
function compareArrays(actual, expected, tolerance) {
  expect(actual.length === expected.length, `length ${actual.length} vs ${expected.length}`);
  let maxAbs = 0, maxRel = 0, worstRatio = 0, worstIndex = -1;
  for (let i = 0; i < expected.length; i++) {
    const e = expected[i];
    const err = Math.abs(actual[i] - e);
    if (!(err === err)) return { maxAbs: NaN, maxRel: NaN, worstRatio: Infinity, worstIndex: i };
    maxAbs = Math.max(maxAbs, err);
    if (e !== 0) maxRel = Math.max(maxRel, err / Math.abs(e));
    const ratio = err / (tolerance.abs + tolerance.rel * Math.abs(e));
    if (ratio > worstRatio) {
      worstRatio = ratio;
      worstIndex = i;
    }
  }
  return { maxAbs, maxRel, worstRatio, worstIndex };
}

function expectMatches(actual, expected, tolerance, label) {
  const r = compareArrays(actual, expected, tolerance);
  expect(r.worstRatio <= 1, `${label}: worst element ${r.worstIndex} at ${(r.worstRatio * 100).toFixed(1)}% of ` +
    `tolerance (abs ${r.maxAbs.toExponential(2)}, rel ${r.maxRel.toExponential(2)})`);
  return r;
}

async function run() {
  let failed = 0;
  for (const c of cases) {
    process.stdout.write(`RUN  ${c.name}\n`);
    const t0 = Date.now();
    try {
      await c.fn();
      process.stdout.write(`PASS ${c.name} (${Date.now() - t0} ms)\n`);
    } catch (err) {
      failed++;
      process.stdout.write(`FAIL ${c.name}: ${err && err.stack ? err.stack : err}\n`);
    }
  }
  for (const hook of afterAllHooks) await hook();
  process.stdout.write(`${cases.length - failed} passed, ${failed} failed\n`);
  process.exitCode = failed ? 1 : 0;
}

module.exports = { describe, it, afterAll, expect, expectThrows, compareArrays, expectMatches, run };
