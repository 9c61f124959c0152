"use strict";
/*
 * hip/acceleration.js -- session-scoped state of the HIP execution provider.
 *
 * Mirrors packages/engine/src/runner/wasm/acceleration.ts for the HIP runner:
 *   registerWasmExecutionProvider 61-63       registerHipExecutionProvider
 *   wasmExecutionProviderStats 65-91          hipExecutionProviderStats
 *   shutdownWasmExecutionProvider 93-112      shutdownHipExecutionProvider
 *   wasmProjectionBatchingEnabled 114-116     hipProjectionBatchingEnabled
 *   wasmResidentWeightCacheEnabled 118-120    hipResidentWeightCacheEnabled
 *   wasmExecutionProviderEnabled 122-124      hipExecutionProviderEnabled
 *   readWasmWeightHandle 164-201              readHipWeightHandle
 *
 * A session (ModelSession, runtime.ts) is used through the members the WASM
 * provider uses: hasProvider(name), provider(name).options,
 * setExecutionProviderStatsProvider(fn, name), getTensor(name) and
 * tensorReader.readTensorBytes(name).  Handles live in HBM; the cache maps
 * tensor names to them, shares a pending upload, and counts hits and misses.
 * A tensor the runner cannot hold (another block type, no GPU) resolves to
 * undefined, so the caller falls back to the WASM runner.
 */

const path = require("path");

let kernels = require(path.join(__dirname, "..", "hip-kernels.js"));

const hipWeightCaches = new WeakMap();
let supportPromise;

/* Replaces the runner module (tests drive the dispatch with a stand-in). */
function setHipKernels(module) {
  kernels = module;
  supportPromise = undefined;
}

function hipKernels() {
  return kernels;
}

function hipSupport() {
  if (!supportPromise) {
    supportPromise = Promise.resolve(kernels.checkHipSupport());
  }
  return supportPromise;
}

function providerOptions(session) {
  const provider = typeof session.provider === "function" ? session.provider("hip") : undefined;
  return (provider && provider.options) || {};
}

function hipExecutionProviderEnabled(session) {
  return typeof session.hasProvider === "function" && session.hasProvider("hip");
}

/* On by default: HBM holds every layer, so the cache has no budget. */
function hipResidentWeightCacheEnabled(session) {
  return hipExecutionProviderEnabled(session) && providerOptions(session).residentWeightCache !== false;
}

function hipProjectionBatchingEnabled(session) {
  return hipResidentWeightCacheEnabled(session) && providerOptions(session).projectionBatching !== false;
}

function ensureHipWeightCache(session) {
  let cache = hipWeightCaches.get(session);
  if (!cache) {
    cache = { handles: new Map(), pending: new Map(), declined: new Set(), bytes: 0, hits: 0, misses: 0, generation: 0 };
    hipWeightCaches.set(session, cache);
  }
  return cache;
}

function registerHipExecutionProvider(session) {
  session.setExecutionProviderStatsProvider(() => hipExecutionProviderStats(session), "hip");
}

function hipExecutionProviderStats(session) {
  const cache = hipWeightCaches.get(session);
  return {
    hipResidentWeightCacheEnabled: hipResidentWeightCacheEnabled(session),
    hipResidentWeightCacheCount: cache ? cache.handles.size : 0,
    hipResidentWeightCacheBytes: cache ? cache.bytes : 0,
    hipResidentWeightCacheHits: cache ? cache.hits : 0,
    hipResidentWeightCacheMisses: cache ? cache.misses : 0,
    hipResidentWeightCacheDeclined: cache ? cache.declined.size : 0,
  };
}

function shutdownHipExecutionProvider(session) {
  const cache = hipWeightCaches.get(session);
  if (cache) {
    cache.generation += 1; // uploads still in flight release their handle on arrival
    for (const handle of cache.handles.values()) {
      kernels.releaseHipQuantizedWeightHandle(handle);
    }
    cache.handles.clear();
    cache.pending.clear();
    cache.declined.clear();
    cache.bytes = 0;
  }
}

/* The HBM-resident handle of tensor `name`, uploaded on first use; undefined
 * when the cache is off, the GPU is unavailable or the runner does not
 * implement the block type.  Shape errors throw, as createWasmQuantizedWeightHandle's do. */
async function readHipWeightHandle(session, name, type, inputSize, rowCount) {
  if (!hipResidentWeightCacheEnabled(session)) {
    return undefined;
  }
  const cache = ensureHipWeightCache(session);
  const cached = cache.handles.get(name);
  if (cached) {
    cache.hits += 1;
    return cached;
  }
  if (cache.declined.has(name)) {
    cache.hits += 1;
    return undefined;
  }
  const pending = cache.pending.get(name);
  if (pending) {
    cache.hits += 1;
    return pending;
  }
  cache.misses += 1;
  const generation = cache.generation;
  const pendingRead = (async () => {
    if (!kernels.quantizedTypeId(type) || !(await hipSupport()).available) {
      if (cache.generation === generation) {
        cache.declined.add(name);
      }
      return undefined;
    }
    const bytes = await session.tensorReader.readTensorBytes(name);
    const handle = await kernels.createHipQuantizedWeightHandle(type, bytes, inputSize, rowCount);
    if (cache.generation !== generation) {
      // shutdownHipExecutionProvider ran while this upload was pending
      if (handle) {
        kernels.releaseHipQuantizedWeightHandle(handle);
      }
      return undefined;
    }
    if (!handle) {
      cache.declined.add(name);
      return undefined;
    }
    cache.handles.set(name, handle);
    cache.bytes += handle.byteLength;
    return handle;
  })();
  cache.pending.set(name, pendingRead);
  try {
    return await pendingRead;
  } finally {
    if (cache.pending.get(name) === pendingRead) {
      cache.pending.delete(name);
    }
  }
}

/* Puts handles uploaded by the file -> HBM loader (HipGgufWeights.upload of
 * hip-kernels.js) into the session cache, so readHipWeightHandle finds them
 * without a JS copy of the tensor bytes.  Names the loader declined are
 * remembered as declined. */
function adoptHipWeightHandles(session, handles) {
  const cache = ensureHipWeightCache(session);
  for (const [name, handle] of handles) {
    if (handle) {
      if (!cache.handles.has(name)) {
        cache.handles.set(name, handle);
        cache.bytes += handle.byteLength;
      }
    } else {
      cache.declined.add(name);
    }
  }
}

module.exports = {
  adoptHipWeightHandles,
  hipExecutionProviderEnabled,
  hipExecutionProviderStats,
  hipKernels,
  hipProjectionBatchingEnabled,
  hipResidentWeightCacheEnabled,
  readHipWeightHandle,
  registerHipExecutionProvider,
  setHipKernels,
  shutdownHipExecutionProvider,
};
