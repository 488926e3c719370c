// Native key -> bytes KV relay over TCP: server, pooled client, CRC-32.
//
// The wire protocol of the reference's cross-node transport
// (connector/tcpkv.py:9-17), little-endian, any number of requests per
// connection:
//   push  'P' klen:i32 key n:i64 crc:u32 data  -> "OK" | "ER" (crc mismatch, blob dropped)
//   take  'W' klen:i32 key wait_ms:i32          -> n:i64 crc:u32 data; n = -1 if absent
//   stats 'S'                                   -> n:i64 json
// crc is zlib's CRC-32 of the data (0 = unchecked), checked by the server on
// arrival and by the client on delivery, so a take returns the pushed bytes or
// fails. A native client speaks to the reference's Python relay and the other
// way round.
//
// Host code only (no HIP): a relay can run on a node without a GPU. Built with
// g++ into librngdpd_net.so; declared in include/rngdpd_net.h.

#include "rngdpd_net.h"

#include <arpa/inet.h>
#include <errno.h>
#include <fcntl.h>
#include <netdb.h>
#include <netinet/in.h>
#include <netinet/tcp.h>
#include <poll.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/socket.h>
#include <sys/uio.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

// ---- CRC-32 (reflected polynomial 0xEDB88320, zlib's) ------------------------
// Slicing by 16: table k maps a byte to its CRC contribution k bytes further
// along, so 16 input bytes fold into the state with 16 independent lookups.
struct CrcTables {
  uint32_t t[16][256];
  CrcTables() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int b = 0; b < 8; ++b) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
      t[0][i] = c;
    }
    for (int k = 1; k < 16; ++k)
      for (int i = 0; i < 256; ++i) t[k][i] = (t[k - 1][i] >> 8) ^ t[0][t[k - 1][i] & 0xff];
  }
};

const CrcTables& tables() {
  static const CrcTables T;
  return T;
}

// Raw update of the (inverted) CRC state over n bytes.
uint32_t crc_raw(uint32_t s, const uint8_t* p, size_t n) {
  const auto& T = tables().t;
  while (n >= 16) {
    uint32_t w[4];
    memcpy(w, p, 16);                 // little-endian host
    w[0] ^= s;
    s = T[15][w[0] & 0xff] ^ T[14][(w[0] >> 8) & 0xff] ^ T[13][(w[0] >> 16) & 0xff] ^
        T[12][w[0] >> 24] ^ T[11][w[1] & 0xff] ^ T[10][(w[1] >> 8) & 0xff] ^
        T[9][(w[1] >> 16) & 0xff] ^ T[8][w[1] >> 24] ^ T[7][w[2] & 0xff] ^
        T[6][(w[2] >> 8) & 0xff] ^ T[5][(w[2] >> 16) & 0xff] ^ T[4][w[2] >> 24] ^
        T[3][w[3] & 0xff] ^ T[2][(w[3] >> 8) & 0xff] ^ T[1][(w[3] >> 16) & 0xff] ^
        T[0][w[3] >> 24];
    p += 16;
    n -= 16;
  }
  while (n--) s = (s >> 8) ^ T[0][(s ^ *p++) & 0xff];
  return s;
}

uint32_t crc32_update(uint32_t crc, const void* p, size_t n) {
  return ~crc_raw(~crc, static_cast<const uint8_t*>(p), n);
}

// ---- socket helpers ------------------------------------------------------------
int send_all(int fd, const void* p, size_t n) {
  const char* c = static_cast<const char*>(p);
  while (n) {
    const ssize_t k = send(fd, c, n, MSG_NOSIGNAL);
    if (k < 0) {
      if (errno == EINTR) continue;
      return -1;
    }
    c += k;
    n -= (size_t)k;
  }
  return 0;
}

// writev of every byte of the iovecs (advanced in place).
int send_iov(int fd, std::vector<iovec>& iov) {
  size_t first = 0;
  while (first < iov.size()) {
    msghdr m{};
    m.msg_iov = iov.data() + first;
    m.msg_iovlen = std::min<size_t>(iov.size() - first, 1024);
    ssize_t k = sendmsg(fd, &m, MSG_NOSIGNAL);
    if (k < 0) {
      if (errno == EINTR) continue;
      return -1;
    }
    while (k > 0 && first < iov.size()) {
      if ((size_t)k >= iov[first].iov_len) {
        k -= (ssize_t)iov[first].iov_len;
        ++first;
      } else {
        iov[first].iov_base = static_cast<char*>(iov[first].iov_base) + k;
        iov[first].iov_len -= (size_t)k;
        k = 0;
      }
    }
    while (first < iov.size() && iov[first].iov_len == 0) ++first;
  }
  return 0;
}

// 1 on success, 0 if the peer closed before the first byte, -1 on error/short.
int recv_exact(int fd, void* p, size_t n) {
  char* c = static_cast<char*>(p);
  size_t got = 0;
  while (got < n) {
    const ssize_t k = recv(fd, c + got, n - got, 0);
    if (k == 0) return got == 0 ? 0 : -1;
    if (k < 0) {
      if (errno == EINTR) continue;
      return -1;
    }
    got += (size_t)k;
  }
  return 1;
}

void no_delay(int fd) {
  int one = 1;
  setsockopt(fd, IPPROTO_TCP, TCP_NODELAY, &one, sizeof one);
}

constexpr int32_t kMaxKey = 1 << 20;
constexpr int64_t kMaxBlob = int64_t(64) << 30;

// ---- server --------------------------------------------------------------------
struct Entry {
  std::vector<char> data;
  uint32_t crc;
  std::chrono::steady_clock::time_point t;
};

struct Server {
  int lfd = -1;
  int port = 0;
  std::atomic<double> ttl_s{900.0};
  std::atomic<bool> stop{false};
  std::mutex mu;
  std::condition_variable cv;
  std::unordered_map<std::string, Entry> store;
  uint64_t pushed = 0, taken = 0, expired = 0, crc_errors = 0, bytes_in = 0, bytes_out = 0;
  std::set<int> conns;                 // open connection sockets (guarded by mu)
  std::atomic<int> live{0};            // connection threads still running
  std::thread acceptor;

  void expire() {
    const auto now = std::chrono::steady_clock::now();
    const double ttl = ttl_s.load();
    std::lock_guard<std::mutex> g(mu);
    for (auto it = store.begin(); it != store.end();) {
      if (std::chrono::duration<double>(now - it->second.t).count() > ttl) {
        it = store.erase(it);
        ++expired;
      } else {
        ++it;
      }
    }
  }

  std::string stats_json() {
    std::lock_guard<std::mutex> g(mu);
    uint64_t held = 0;
    for (auto& kv : store) held += kv.second.data.size();
    char buf[512];
    snprintf(buf, sizeof buf,
             "{\"pushed\": %llu, \"taken\": %llu, \"expired\": %llu, \"crc_errors\": %llu, "
             "\"bytes_in\": %llu, \"bytes_out\": %llu, \"keys\": %zu, \"bytes_held\": %llu}",
             (unsigned long long)pushed, (unsigned long long)taken,
             (unsigned long long)expired, (unsigned long long)crc_errors,
             (unsigned long long)bytes_in, (unsigned long long)bytes_out, store.size(),
             (unsigned long long)held);
    return buf;
  }

  void serve(int fd) {
    for (;;) {
      char op;
      if (recv_exact(fd, &op, 1) != 1) break;
      if (op == 'S') {
        const std::string js = stats_json();
        const int64_t n = (int64_t)js.size();
        if (send_all(fd, &n, 8) || send_all(fd, js.data(), js.size())) break;
        continue;
      }
      if (op != 'P' && op != 'W') break;             // unknown op: drop the connection
      int32_t klen;
      if (recv_exact(fd, &klen, 4) != 1 || klen < 0 || klen > kMaxKey) break;
      std::string key((size_t)klen, '\0');
      if (klen && recv_exact(fd, &key[0], (size_t)klen) != 1) break;
      if (op == 'P') {
        int64_t n;
        uint32_t crc;
        if (recv_exact(fd, &n, 8) != 1 || recv_exact(fd, &crc, 4) != 1) break;
        if (n < 0 || n > kMaxBlob) break;
        std::vector<char> data((size_t)n);
        if (n && recv_exact(fd, data.data(), (size_t)n) != 1) break;
        if (crc && crc32_update(0, data.data(), data.size()) != crc) {
          {
            std::lock_guard<std::mutex> g(mu);
            ++crc_errors;
          }
          if (send_all(fd, "ER", 2)) break;
          continue;
        }
        {
          std::lock_guard<std::mutex> g(mu);
          bytes_in += (uint64_t)n;
          ++pushed;
          store[key] = Entry{std::move(data), crc, std::chrono::steady_clock::now()};
        }
        cv.notify_all();
        if (send_all(fd, "OK", 2)) break;
      } else {
        int32_t wait_ms;
        if (recv_exact(fd, &wait_ms, 4) != 1) break;
        const auto deadline =
            std::chrono::steady_clock::now() + std::chrono::milliseconds(std::max(0, wait_ms));
        Entry e;
        bool found = false;
        {
          std::unique_lock<std::mutex> g(mu);
          cv.wait_until(g, deadline, [&] { return stop.load() || store.count(key) > 0; });
          auto it = store.find(key);
          if (it != store.end()) {
            e = std::move(it->second);
            store.erase(it);
            found = true;
            ++taken;
            bytes_out += e.data.size();
          }
        }
        if (!found) {
          const int64_t n = -1;
          const uint32_t crc = 0;
          if (send_all(fd, &n, 8) || send_all(fd, &crc, 4)) break;
        } else {
          const int64_t n = (int64_t)e.data.size();
          char hdr[12];
          memcpy(hdr, &n, 8);
          memcpy(hdr + 8, &e.crc, 4);
          std::vector<iovec> iov{{hdr, 12}, {e.data.data(), e.data.size()}};
          if (send_iov(fd, iov)) break;
        }
      }
    }
    {
      std::lock_guard<std::mutex> g(mu);
      conns.erase(fd);
    }
    close(fd);
  }

  void accept_loop(std::shared_ptr<Server> self) {
    while (!stop.load()) {
      pollfd p{lfd, POLLIN, 0};
      const int r = poll(&p, 1, 500);
      if (r == 0) {
        expire();
        continue;
      }
      if (r < 0) {
        if (errno == EINTR) continue;
        break;
      }
      const int fd = accept(lfd, nullptr, nullptr);
      if (fd < 0) continue;
      no_delay(fd);
      {
        std::lock_guard<std::mutex> g(mu);
        if (stop.load()) {
          close(fd);
          break;
        }
        conns.insert(fd);
      }
      ++live;
      std::thread([self, fd] {
        self->serve(fd);
        --self->live;
      }).detach();
    }
  }
};

struct ServerHandle {
  std::shared_ptr<Server> s;
};

// ---- client --------------------------------------------------------------------
struct Client {
  std::string host;
  int port = 0;
  double connect_timeout = 10.0;
  std::mutex mu;
  std::vector<int> idle;               // LIFO: the most recently used connection first
  std::string stash_key;               // a blob too large for the last take_into
  std::vector<char> stash;

  int dial() {
    addrinfo hints{}, *res = nullptr;
    hints.ai_family = AF_UNSPEC;
    hints.ai_socktype = SOCK_STREAM;
    char ps[16];
    snprintf(ps, sizeof ps, "%d", port);
    const int gr = getaddrinfo(host.c_str(), ps, &hints, &res);
    if (gr != 0) return fail(PDK_NET_ECONN, "resolve %s: %s", host.c_str(), gai_strerror(gr));
    int fd = -1;
    for (addrinfo* a = res; a; a = a->ai_next) {
      fd = socket(a->ai_family, a->ai_socktype, a->ai_protocol);
      if (fd < 0) continue;
      const int fl = fcntl(fd, F_GETFL, 0);
      fcntl(fd, F_SETFL, fl | O_NONBLOCK);
      int r = connect(fd, a->ai_addr, a->ai_addrlen);
      if (r < 0 && errno == EINPROGRESS) {
        pollfd p{fd, POLLOUT, 0};
        r = poll(&p, 1, (int)(connect_timeout * 1000));
        int err = 0;
        socklen_t len = sizeof err;
        if (r == 1 && getsockopt(fd, SOL_SOCKET, SO_ERROR, &err, &len) == 0 && err == 0) r = 0;
        else r = -1;
      }
      if (r == 0) {
        fcntl(fd, F_SETFL, fl);
        no_delay(fd);
        break;
      }
      close(fd);
      fd = -1;
    }
    freeaddrinfo(res);
    if (fd < 0) return fail(PDK_NET_ECONN, "connect %s:%d failed", host.c_str(), port);
    return fd;
  }

  int borrow() {
    {
      std::lock_guard<std::mutex> g(mu);
      if (!idle.empty()) {
        const int fd = idle.back();
        idle.pop_back();
        return fd;
      }
    }
    return dial();
  }

  void give_back(int fd) {
    std::lock_guard<std::mutex> g(mu);
    idle.push_back(fd);
  }
};

}  // namespace

extern "C" {

const char* pdk_net_last_error(void) { return g_err; }

uint32_t pdk_crc32(uint32_t crc, const void* data, size_t n) {
  return crc32_update(crc, data, n);
}

int pdk_tcp_server_start(const char* host, int port, double ttl_s, void** out) {
  if (!out || port < 0 || port > 65535) return fail(PDK_NET_EINVAL, "bad arguments");
  *out = nullptr;
  auto s = std::make_shared<Server>();
  if (ttl_s >= 0) s->ttl_s = ttl_s;
  s->lfd = socket(AF_INET, SOCK_STREAM, 0);
  if (s->lfd < 0) return fail(PDK_NET_ECONN, "socket: %s", strerror(errno));
  int one = 1;
  setsockopt(s->lfd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof one);
  sockaddr_in a{};
  a.sin_family = AF_INET;
  a.sin_port = htons((uint16_t)port);
  const char* h = (host && *host) ? host : "0.0.0.0";
  if (inet_pton(AF_INET, h, &a.sin_addr) != 1) {
    close(s->lfd);
    return fail(PDK_NET_EINVAL, "bind address %s is not an IPv4 address", h);
  }
  if (bind(s->lfd, (sockaddr*)&a, sizeof a) < 0 || listen(s->lfd, 64) < 0) {
    const int e = errno;
    close(s->lfd);
    return fail(PDK_NET_ECONN, "bind/listen %s:%d: %s", h, port, strerror(e));
  }
  socklen_t len = sizeof a;
  getsockname(s->lfd, (sockaddr*)&a, &len);
  s->port = ntohs(a.sin_port);
  s->acceptor = std::thread([s] { s->accept_loop(s); });
  *out = new ServerHandle{s};
  return PDK_NET_OK;
}

int pdk_tcp_server_port(void* server) {
  return server ? static_cast<ServerHandle*>(server)->s->port : PDK_NET_EINVAL;
}

int pdk_tcp_server_set_ttl(void* server, double ttl_s) {
  if (!server || ttl_s < 0) return fail(PDK_NET_EINVAL, "bad arguments");
  static_cast<ServerHandle*>(server)->s->ttl_s = ttl_s;
  return PDK_NET_OK;
}

int64_t pdk_tcp_server_stats(void* server, char* buf, size_t cap) {
  if (!server || !buf) return fail(PDK_NET_EINVAL, "bad arguments");
  const std::string js = static_cast<ServerHandle*>(server)->s->stats_json();
  if (js.size() + 1 > cap) return fail(PDK_NET_ENOSPC, "stats need %zu bytes", js.size() + 1);
  memcpy(buf, js.c_str(), js.size() + 1);
  return (int64_t)js.size();
}

int pdk_tcp_server_stop(void* server) {
  if (!server) return fail(PDK_NET_EINVAL, "null server");
  auto* h = static_cast<ServerHandle*>(server);
  Server& s = *h->s;
  {
    std::lock_guard<std::mutex> g(s.mu);
    s.stop = true;
    for (int fd : s.conns) shutdown(fd, SHUT_RDWR);   // wake blocked receives
  }
  s.cv.notify_all();                                  // wake waiting takes
  if (s.acceptor.joinable()) s.acceptor.join();
  close(s.lfd);
  for (int i = 0; i < 500 && s.live.load() > 0; ++i)
    std::this_thread::sleep_for(std::chrono::milliseconds(10));
  delete h;                             // threads still running keep the state alive
  return PDK_NET_OK;
}

int pdk_tcp_client_open(const char* host, int port, double connect_timeout, void** out) {
  if (!out || !host || port <= 0 || port > 65535) return fail(PDK_NET_EINVAL, "bad arguments");
  auto* c = new Client;
  c->host = host;
  c->port = port;
  c->connect_timeout = connect_timeout > 0 ? connect_timeout : 10.0;
  *out = c;
  return PDK_NET_OK;
}

int pdk_tcp_client_idle(void* client) {
  if (!client) return PDK_NET_EINVAL;
  auto* c = static_cast<Client*>(client);
  std::lock_guard<std::mutex> g(c->mu);
  return (int)c->idle.size();
}

int pdk_tcp_client_close(void* client) {
  if (!client) return fail(PDK_NET_EINVAL, "null client");
  auto* c = static_cast<Client*>(client);
  for (int fd : c->idle) close(fd);
  delete c;
  return PDK_NET_OK;
}

int pdk_tcp_push(void* client, const char* key, const void* const* parts, const size_t* lens,
                 int nparts, int crc_on) {
  if (!client || !key || nparts < 0 || (nparts && (!parts || !lens)))
    return fail(PDK_NET_EINVAL, "bad arguments");
  auto* c = static_cast<Client*>(client);
  const size_t klen = strlen(key);
  if (klen > (size_t)kMaxKey) return fail(PDK_NET_EINVAL, "key too long");
  uint64_t n = 0;
  uint32_t crc = 0;
  for (int i = 0; i < nparts; ++i) {
    n += lens[i];
    if (crc_on) crc = crc32_update(crc, parts[i], lens[i]);
  }
  // crc 0 means "unchecked" on the wire; a blob whose CRC-32 is 0 goes unchecked too.
  char hdr[1 + 4 + 8 + 4];
  const int32_t kl = (int32_t)klen;
  const int64_t nn = (int64_t)n;
  std::vector<iovec> iov;
  iov.reserve(3 + (size_t)nparts);
  hdr[0] = 'P';
  memcpy(hdr + 1, &kl, 4);
  iov.push_back({hdr, 5});
  iov.push_back({const_cast<char*>(key), klen});
  char tail[12];
  memcpy(tail, &nn, 8);
  memcpy(tail + 8, &crc, 4);
  iov.push_back({tail, 12});
  for (int i = 0; i < nparts; ++i)
    if (lens[i]) iov.push_back({const_cast<void*>(parts[i]), lens[i]});
  const int fd = c->borrow();
  if (fd < 0) return fd;
  char ack[2];
  if (send_iov(fd, iov) || recv_exact(fd, ack, 2) != 1) {
    close(fd);
    return fail(PDK_NET_ECONN, "push %s: connection lost", key);
  }
  c->give_back(fd);
  if (ack[0] != 'O' || ack[1] != 'K')
    return fail(PDK_NET_EIO, "push %s: server rejected the blob (crc mismatch)", key);
  return PDK_NET_OK;
}

int pdk_tcp_take(void* client, const char* key, int wait_ms, void* dst, size_t cap,
                 int64_t* n_out, int crc_check) {
  if (!client || !key || !n_out || wait_ms < 0 || (cap && !dst))
    return fail(PDK_NET_EINVAL, "bad arguments");
  auto* c = static_cast<Client*>(client);
  *n_out = -1;
  {
    std::lock_guard<std::mutex> g(c->mu);
    if (!c->stash.empty() || !c->stash_key.empty()) {
      if (c->stash_key == key) {
        *n_out = (int64_t)c->stash.size();
        if (c->stash.size() > cap)
          return fail(PDK_NET_ENOSPC, "take %s: %zu bytes do not fit %zu", key, c->stash.size(),
                      cap);
        if (!c->stash.empty()) memcpy(dst, c->stash.data(), c->stash.size());
        c->stash.clear();
        c->stash_key.clear();
        return PDK_NET_OK;
      }
    }
  }
  const size_t klen = strlen(key);
  if (klen > (size_t)kMaxKey) return fail(PDK_NET_EINVAL, "key too long");
  char hdr[5];
  hdr[0] = 'W';
  const int32_t kl = (int32_t)klen;
  memcpy(hdr + 1, &kl, 4);
  std::vector<iovec> iov{{hdr, 5}, {const_cast<char*>(key), klen}, {&wait_ms, 4}};
  const int fd = c->borrow();
  if (fd < 0) return fd;
  int64_t n;
  uint32_t crc;
  if (send_iov(fd, iov) || recv_exact(fd, &n, 8) != 1 || recv_exact(fd, &crc, 4) != 1) {
    close(fd);
    return fail(PDK_NET_ECONN, "take %s: connection lost", key);
  }
  if (n < 0) {
    c->give_back(fd);
    return fail(PDK_NET_ETIMEDOUT, "pull timeout: %s", key);
  }
  std::vector<char> big;
  char* into = static_cast<char*>(dst);
  if ((uint64_t)n > cap) {
    big.resize((size_t)n);
    into = big.data();
  }
  if (n && recv_exact(fd, into, (size_t)n) != 1) {
    close(fd);
    return fail(PDK_NET_ECONN, "take %s: connection lost after the header", key);
  }
  c->give_back(fd);
  *n_out = n;
  if (crc && crc_check && crc32_update(0, into, (size_t)n) != crc)
    return fail(PDK_NET_EIO, "tcpkv take %s: crc mismatch on delivery", key);
  if (!big.empty() || (uint64_t)n > cap) {
    std::lock_guard<std::mutex> g(c->mu);
    c->stash_key = key;
    c->stash = std::move(big);
    return fail(PDK_NET_ENOSPC, "take %s: %lld bytes do not fit %zu (kept for the next take)",
                key, (long long)n, cap);
  }
  return PDK_NET_OK;
}

int64_t pdk_tcp_stats(void* client, char* buf, size_t cap) {
  if (!client || !buf) return fail(PDK_NET_EINVAL, "bad arguments");
  auto* c = static_cast<Client*>(client);
  const int fd = c->borrow();
  if (fd < 0) return fd;
  int64_t n;
  if (send_all(fd, "S", 1) || recv_exact(fd, &n, 8) != 1 || n < 0 || n > (1 << 20)) {
    close(fd);
    return fail(PDK_NET_ECONN, "stats: connection lost");
  }
  std::vector<char> js((size_t)n);
  if (n && recv_exact(fd, js.data(), (size_t)n) != 1) {
    close(fd);
    return fail(PDK_NET_ECONN, "stats: connection lost");
  }
  c->give_back(fd);
  if ((size_t)n + 1 > cap) return fail(PDK_NET_ENOSPC, "stats need %lld bytes", (long long)n + 1);
  memcpy(buf, js.data(), (size_t)n);
  buf[n] = '\0';
  return n;
}

}  // extern "C"
