// Loads the N-API addon. There is no fallback: without the built addon (and the HIP library
// it links) every entry point of this package fails here, by name.
'use strict';

const path = require('path');

const ADDON = path.join(__dirname, 'eg_napi.node');

let native;
try {
  native = require(ADDON);
} catch (err) {
  const e = new Error(`enargeia_amd: cannot load ${ADDON} (build it with python -m enargeia_amd.build): ${err.message}`);
  e.code = 'EG_NATIVE_MISSING';
  throw e;
}

module.exports = native;
