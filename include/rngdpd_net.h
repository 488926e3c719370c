/* librngdpd_net: the cross-node `tcp` KV transport as native code.
 *
 * Host-only C ABI (no GPU runtime), built with g++ into librngdpd_net.so so
 * that a relay can run on a node without a GPU. It replaces the reference's
 * Python relay and client (connector/tcpkv.py) with the same wire protocol
 * (connector/tcpkv.py:9-17), so native and Python peers interoperate:
 *
 *   push  'P' klen:i32 key n:i64 crc:u32 data  -> "OK" | "ER"
 *   take  'W' klen:i32 key wait_ms:i32          -> n:i64 crc:u32 data (n = -1: absent)
 *   stats 'S'                                   -> n:i64 json
 *
 * little-endian; crc = zlib CRC-32 of the data, 0 = unchecked. Every call
 * returns 0 or a negative errno-style code; pdk_net_last_error() holds the
 * calling thread's message.
 */
#ifndef RNGDPD_NET_H
#define RNGDPD_NET_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PDK_NET_OK 0
#define PDK_NET_EIO (-5)         /* crc mismatch (push rejected, or on delivery) */
#define PDK_NET_EINVAL (-22)     /* bad argument                                  */
#define PDK_NET_ENOSPC (-28)     /* blob larger than the buffer (kept for a retry) */
#define PDK_NET_ETIMEDOUT (-110) /* take: nothing under the key within wait_ms    */
#define PDK_NET_ECONN (-111)     /* resolve / connect / connection lost           */

const char* pdk_net_last_error(void);

/* zlib's crc32(crc, data, n): CRC-32 with the reflected polynomial 0xEDB88320,
 * chainable (pdk_crc32(pdk_crc32(0, a), b) == CRC-32 of a then b). The blob
 * checksum of connector/tcpkv.py:138,184 (zlib.crc32). */
uint32_t pdk_crc32(uint32_t crc, const void* data, size_t n);

/* ---- relay server (TcpKVServer, connector/tcpkv.py:48-151) ----------------------
 * In-memory key -> blob store behind an IPv4 TCP port (port 0: the OS picks;
 * pdk_tcp_server_port tells which). A take waits up to wait_ms for the key and
 * removes it; a blob nobody takes within ttl_s (900 s when ttl_s < 0) is
 * dropped, checked every 0.5 s. One thread per connection. */
int pdk_tcp_server_start(const char* host, int port, double ttl_s, void** server);
int pdk_tcp_server_port(void* server);
int pdk_tcp_server_set_ttl(void* server, double ttl_s);
/* JSON counters {pushed, taken, expired, crc_errors, bytes_in, bytes_out, keys,
 * bytes_held} into buf; returns the length. */
int64_t pdk_tcp_server_stats(void* server, char* buf, size_t cap);
/* Stops accepting, wakes waiting takes, closes connections, frees the handle. */
int pdk_tcp_server_stop(void* server);

/* ---- pooled client (TcpKVClient, connector/tcpkv.py:154-227) --------------------
 * Persistent connections, borrowed one per call (thread-safe) and kept open
 * afterwards; a connection whose call failed is closed, never reused. */
int pdk_tcp_client_open(const char* host, int port, double connect_timeout, void** client);
int pdk_tcp_client_idle(void* client);           /* connections in the pool */
int pdk_tcp_client_close(void* client);
/* Push the concatenation of nparts buffers under key, one send of all of them;
 * crc_on computes the CRC-32 (else 0, unchecked). PDK_NET_EIO if the server
 * rejected the blob. */
int pdk_tcp_push(void* client, const char* key, const void* const* parts,
                 const size_t* lens, int nparts, int crc_on);
/* Take the blob under key into dst (cap bytes), waiting up to wait_ms; *n_out
 * = its size. PDK_NET_ETIMEDOUT when absent; PDK_NET_EIO on a crc mismatch
 * (crc_check); PDK_NET_ENOSPC when it does not fit: the blob is kept by the
 * client and the next take of the same key (with cap >= *n_out) returns it
 * without a network round trip. */
int pdk_tcp_take(void* client, const char* key, int wait_ms, void* dst, size_t cap,
                 int64_t* n_out, int crc_check);
/* The server's JSON counters into buf; returns the length. */
int64_t pdk_tcp_stats(void* client, char* buf, size_t cap);

#ifdef __cplusplus
}
#endif

#endif /* RNGDPD_NET_H */
