'use strict';
// HTTP client of the engine (Node.js http module; the server is quipullm's, on the same PC).  JSON requests with
// a time limit, and byte ranges of a file (the reference engine fetches tensors with Range requests,
// web/js/weights.js:51).
const http = require('http');
const { URL } = require('url');

// JSON request: metodo 'GET' or 'POST' (with cuerpo), rejected after ms milliseconds (0: no limit).  Resolves to the
// parsed body; an HTTP status >= 400 rejects with an Error carrying `codigo`.
function pedirJSON(url, metodo, cuerpo, ms) {
  return new Promise(function (resolve, reject) {
    const u = new URL(url);
    const datos = cuerpo === undefined ? null : Buffer.from(JSON.stringify(cuerpo));
    const req = http.request({ hostname: u.hostname, port: u.port, path: u.pathname + u.search, method: metodo,
      headers: datos ? { 'Content-Type': 'application/json', 'Content-Length': datos.length } : {} }, function (res) {
      const trozos = [];
      res.on('data', function (c) { trozos.push(c); });
      res.on('end', function () {
        const texto = Buffer.concat(trozos).toString('utf8');
        if (res.statusCode >= 400) {
          const e = new Error('HTTP ' + res.statusCode + ' ' + texto.slice(0, 200));
          e.codigo = res.statusCode;
          reject(e);
          return;
        }
        try { resolve(texto ? JSON.parse(texto) : null); } catch (e) { reject(e); }
      });
      res.on('error', reject);
    });
    req.on('error', reject);
    if (ms > 0) req.setTimeout(ms, function () { const e = new Error('timeout'); e.name = 'AbortError'; req.destroy(e); });
    if (datos) req.write(datos);
    req.end();
  });
}

// Bytes [ini, ini + n) of the file at url (one Range request; the server answers 206).
function rango(url, ini, n) {
  return new Promise(function (resolve, reject) {
    const u = new URL(url);
    const req = http.request({ hostname: u.hostname, port: u.port, path: u.pathname + u.search, method: 'GET',
      headers: { Range: 'bytes=' + ini + '-' + (ini + n - 1) } }, function (res) {
      if (res.statusCode !== 206 && res.statusCode !== 200) {
        res.resume();
        reject(new Error('HTTP ' + res.statusCode + ' reading ' + url));
        return;
      }
      const out = Buffer.allocUnsafe(n);
      let got = 0, salto = res.statusCode === 200 ? ini : 0;   // a server without ranges sends the whole file
      let hecho = false;
      res.on('data', function (c) {
        if (hecho) return;
        if (salto) { const s = Math.min(salto, c.length); c = c.subarray(s); salto -= s; }
        const k = Math.min(c.length, n - got);
        c.copy(out, got, 0, k);
        got += k;
        if (got === n && res.statusCode === 200) {
          // the n wanted bytes are in: stop the rest of a whole-file answer instead of streaming it to the end
          hecho = true;
          resolve(out);
          req.destroy();
        }
      });
      res.on('end', function () {
        if (hecho) return;
        if (got !== n) reject(new Error('incomplete range of ' + url + ': ' + got + ' of ' + n + ' bytes'));
        else resolve(out);
      });
      res.on('error', function (e) { if (!hecho) reject(e); });
    });
    req.on('error', reject);
    req.end();
  });
}

const dormir = function (ms) { return new Promise(function (r) { setTimeout(r, ms); }); };

module.exports = { pedirJSON: pedirJSON, rango: rango, dormir: dormir };
