// enargeia_amd for Node: the reference's gpu layer and kernel-op interface for the quantized
// projection path, over HIP on MI355X through the N-API addon (eg_napi.node).
'use strict';

module.exports = Object.assign({}, require('./gpu.js'), require('./kernel.js'), require('./ops.js'),
  require('./decoder.js'), require('./container.js'), {
  native: require('./native.js'),
});
